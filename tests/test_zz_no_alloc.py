"""spruce_kv_summary_noalloc (the allocation-free form of spruce_kv_summary)
against spruce_kv_summary, through the C ABI.

Both entry points run the same kernels, one on a caller workspace and one on
the library's static scratch, so the bar is bit-exact equality of keys,
values, counts and log counts.  Two calls in a row on the shared scratch, the
second with a smaller input (and a padding mask), then a third on the scalar
path (D = 48); then two calls issued back to back on two streams with no host
synchronisation between them, which the library orders on the device.  (The
rejection of shapes above the scratch limit needs no GPU: tests/test_abi.py.)
"""
import pytest
import torch

import spruce_hip
from interfaces.residual_summaries import build_residual_tree_layout
from sparse.summaries import build_kv_summary_table

pytestmark = pytest.mark.gpu
DEV = "cuda"
LIMIT = 64 << 20


def _noalloc(key, value, table, valid=None):
    B, H, _, D = key.shape
    keys = torch.full_like(table.keys, float("nan"))
    values = torch.full_like(table.values, float("nan"))
    counts = torch.full_like(table.counts, float("nan"))
    log_counts = torch.full_like(table.log_counts, float("nan"))
    starts = table.range_starts.contiguous().view(-1)
    ends = table.range_ends.contiguous().view(-1)
    valid_u8 = None if valid is None else valid.to(torch.bool).contiguous().view(torch.uint8)
    with torch.cuda.device(key.device):
        rc = spruce_hip.lib().spruce_kv_summary_noalloc(
            spruce_hip.ptr(key), spruce_hip.strides(key), spruce_hip.ptr(value), spruce_hip.strides(value),
            B, H, key.shape[2], D, spruce_hip.dtype_code(key), spruce_hip.ptr(valid_u8),
            spruce_hip.ptr(starts), spruce_hip.ptr(ends), starts.numel(),
            spruce_hip.ptr(keys), spruce_hip.ptr(values), spruce_hip.ptr(counts), spruce_hip.ptr(log_counts),
            spruce_hip.stream_of(key))
    spruce_hip.check(rc, "spruce_kv_summary_noalloc")
    return keys, values, counts, log_counts


def _inputs(T, H, D, dtype, prototypes, masked, seed):
    gen = torch.Generator().manual_seed(seed)
    key = torch.randn(1, T, H, D, generator=gen).to(dtype).to(DEV).transpose(1, 2)
    value = torch.randn(1, T, H, D, generator=gen).to(dtype).to(DEV).transpose(1, 2)
    valid = None
    if masked:
        valid = torch.ones(1, T, dtype=torch.bool)
        valid[0, : T // 5] = False
        valid = valid.to(DEV)
    layout = build_residual_tree_layout((T + 63) // 64)
    need = spruce_hip.lib().spruce_kv_summary_workspace_bytes(1, H, T, D)
    print(f"case T={T} H={H} D={D} {dtype} P={prototypes} masked={masked} scratch={need} bytes", flush=True)
    assert need <= LIMIT
    table = build_kv_summary_table(key, value, layout, block_size=64, prototypes=prototypes, token_mask=valid)
    return key, value, valid, table


def _check(got, table):
    for name, a, b in zip(("keys", "values", "counts", "log_counts"), got,
                          (table.keys, table.values, table.counts, table.log_counts)):
        assert torch.equal(a, b), name


def _case(T, H, D, dtype, prototypes, masked, seed):
    key, value, valid, table = _inputs(T, H, D, dtype, prototypes, masked, seed)
    got = _noalloc(key, value, table, valid)
    torch.cuda.synchronize()
    _check(got, table)


def test_noalloc_matches_workspace_entry_on_consecutive_calls():
    _case(65536, 4, 128, torch.bfloat16, 4, False, 0)   # cfg3 shape: 32 MiB of scratch
    _case(3000, 2, 128, torch.float16, 2, True, 1)      # smaller, ragged, padding mask
    _case(1000, 3, 48, torch.float32, 1, True, 2)       # scalar chunk path


def test_noalloc_calls_on_two_streams_are_ordered():
    big = _inputs(65536, 4, 128, torch.bfloat16, 4, False, 3)
    small = _inputs(3000, 2, 128, torch.float16, 2, True, 4)
    torch.cuda.synchronize()
    streams = (torch.cuda.Stream(), torch.cuda.Stream())   # default priority
    for order in ((big, small), (small, big)):
        results = []
        for stream, (key, value, valid, table) in zip(streams, order):
            stream.wait_stream(torch.cuda.current_stream())
            with torch.cuda.stream(stream):
                results.append(_noalloc(key, value, table, valid))
        torch.cuda.synchronize()
        for got, (_, _, _, table) in zip(results, order):
            _check(got, table)
