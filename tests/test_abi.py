"""The C ABI library: it loads, exports every symbol include/*.h declares, and
rejects invalid arguments with SPRUCE_EINVAL before touching the GPU (so these
run on a machine without one)."""
import ctypes
import glob
import os
import re

import pytest

import spruce_hip

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _declared_functions():
    names = set()
    for header in glob.glob(os.path.join(ROOT, "include", "*.h")):
        text = open(header).read()
        text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
        names.update(re.findall(r"\b(spruce_\w+)\s*\(", text))
    return sorted(names)


def test_library_is_built_and_exports_every_declared_symbol():
    assert spruce_hip.is_built(), "run __graft_entry__.build() first"
    lib = ctypes.CDLL(spruce_hip.LIB_PATH)
    declared = _declared_functions()
    assert "spruce_sparse_prefill_index" in declared
    missing = [n for n in declared if not hasattr(lib, n)]
    assert not missing, missing


def test_version_string():
    assert "gfx950" in spruce_hip.version()


def _strides(*s):
    return (ctypes.c_int64 * 4)(*s)


def _call_index(D=128, Hq=4, Hkv=2, dtype=0, variant=0, qs=(0, 0, 128, 1), K=1, null_idx=False):
    lib = spruce_hip.lib()
    fake = ctypes.c_void_p(1 << 20)  # never dereferenced: validation fails first
    return lib.spruce_sparse_prefill_index(
        fake, _strides(*qs), fake, _strides(0, 0, 128, 1), fake, _strides(0, 0, 128, 1),
        None if null_idx else fake, _strides(0, 0, 1, 1), K,
        1, Hq, Hkv, 64, D, 0.1, dtype, variant, fake, _strides(0, 128, 512, 1), None)


@pytest.mark.parametrize("kwargs, message", [
    (dict(D=96), "head_dim 64 or 128"),
    (dict(Hq=3, Hkv=2), "divisible"),
    (dict(dtype=7), "dtype"),
    (dict(variant=9), "variant"),
    (dict(qs=(0, 0, 128, 2)), "contiguous final dimension"),
    (dict(qs=(0, 0, 100, 1)), "16-byte aligned"),
    (dict(null_idx=True), "indices"),
])
def test_invalid_arguments_return_einval_with_message(kwargs, message):
    rc = _call_index(**kwargs)
    assert rc == -1
    assert message in spruce_hip.last_error()


def test_packing_and_proto_validation_before_launch():
    lib = spruce_hip.lib()
    fake = ctypes.c_void_p(1 << 20)
    # k_selected 2 cannot hold local window 2 plus one sink block.
    assert lib.spruce_pack_selected_ids(fake, 8, 4, 4, 2, 4, 2, 1, 1, fake, 2, None) == -1
    assert "sink block" in spruce_hip.last_error()
    # out_cols must equal min(k, C + sink + lw + 1) = min(8, 2 + 0 + 2) = 4.
    assert lib.spruce_pack_selected_ids(fake, 4, 4, 4, 2, 4, 8, 1, 0, fake, 8, None) == -1
    assert "4 columns" in spruce_hip.last_error()
    assert lib.spruce_pack_selected_mask(fake, 4, 4, 4, 1, 1, fake, 1, None) == -1
    assert "cannot fit local window" in spruce_hip.last_error()
    assert lib.spruce_proto_pool(fake, _strides(0, 0, 256, 1), 1, 4, 64, 256, 4, 64, 8, 0, fake, None) == -1
    assert "head_dim must be <= 128" in spruce_hip.last_error()
    assert lib.spruce_group_avg_tokens(fake, _strides(0, 0, 128, 1), 1, 6, 64, 128, 4, 0, fake, None) == -1
    assert "not divisible" in spruce_hip.last_error()


def test_tree_merge_levels_validation_before_launch():
    lib = spruce_hip.lib()
    fake = ctypes.c_void_p(1 << 20)
    parents = (ctypes.c_void_p * 2)(fake, fake)
    cases = [((1, 4, 8, 16, 0, 0, parents, 2), "radix must be >= 2"),
             ((1, 4, 0, 16, 2, 0, parents, 2), "P and D must be positive"),
             ((1, 4, 8, 16, 2, 9, parents, 2), "unsupported dtype"),
             ((1, 4, 8, 16, 2, 0, parents, 0), "levels must be in [1, 32]"),
             ((1, 4, 8, 16, 2, 0, (ctypes.c_void_p * 2)(fake, None), 2), "parent level 1 is a null pointer"),
             ((1, 4, 40, 16, 2, 0, parents, 2), "radix * P must be <= 64"),
             # Factors whose int64 product would overflow are rejected before it is formed.
             ((1, 4, 1 << 62, 16, 4, 0, parents, 2), "radix * P must be <= 64"),
             ((1, 4, 1 << 40, 16, 1 << 40, 0, parents, 2), "radix * P must be <= 64"),
             ((1, 4, 8, 1 << 62, 2, 0, parents, 2), "feature dim must be <= 256")]
    for args, message in cases:
        assert lib.spruce_tree_merge_levels(fake, *args, None) == -1, message
        assert message in spruce_hip.last_error(), (message, spruce_hip.last_error())
    assert lib.spruce_tree_merge_level(fake, 1, 4, 1 << 62, 16, 4, 0, fake, None) == -1
    assert "radix * P must be <= 64" in spruce_hip.last_error()
    # Traversal: beam * radix is bounded the same way.
    for beam, radix in ((1 << 62, 4), (4, 1 << 62), (33, 2)):
        assert lib.spruce_tree_traverse(fake, fake, 1, 4, 8, 1, 1, 16, radix, beam, 1.0, fake, 4, 0, None) == -1
        assert "beam * radix must be <= 64" in spruce_hip.last_error()
    assert lib.spruce_tree_traverse(fake, fake, 1, 4, 8, 1, 1, 16, 2, 4, 1.0, fake, 4, 2, None) == -1
    assert "unknown key table layout" in spruce_hip.last_error()


def test_error_codes_map_to_reference_exception_types():
    assert _call_index(D=96) == -1
    with pytest.raises(ValueError, match="head_dim"):
        spruce_hip.check(-1, "spruce_sparse_prefill_index")


def test_kernel_metadata_reports_launch_shape():
    cfg = spruce_hip.launch_config("single_head", 28, 4, 128)
    assert cfg["variant"] == "single_head"
    best = cfg["best_config"]
    # Every query head of the KV group is covered: 7 heads x 64 rows per row.
    assert best["waves_per_workgroup"] * best["workgroups_per_row"] * best["query_rows_per_wave"] >= 7 * 64
    assert spruce_hip.launch_config("single_head_prescale", 8, 2, 64)["best_config"]["prescale_q"]
    # The reference's best_config keys (kernels/seerattention_direct_index_triton.py:419-427),
    # which its profiling scripts serialise.
    assert {"kwargs", "num_warps", "num_stages", "num_ctas"} <= set(best)
    assert isinstance(best["kwargs"], dict) and best["num_warps"] == best["waves_per_workgroup"]
    assert all(isinstance(best[k], int) for k in ("num_warps", "num_stages", "num_ctas"))


def test_noalloc_rejects_shapes_above_the_scratch_limit():
    # spruce_kv_summary_noalloc checks the scratch size before any HIP call, so
    # the fake pointers are never used.
    lib = spruce_hip.lib()
    limit = 64 << 20
    assert lib.spruce_kv_summary_workspace_bytes(1, 8, 131072, 128) > limit
    assert lib.spruce_kv_summary_workspace_bytes(1, 4, 65536, 128) <= limit
    fake = ctypes.c_void_p(1 << 20)
    st = (ctypes.c_int64 * 4)(0, 0, 128, 1)
    rc = lib.spruce_kv_summary_noalloc(fake, st, fake, st, 1, 8, 131072, 128, 0, None, fake, fake, 16,
                                       fake, fake, fake, fake, None)
    assert rc == -1
    assert "above its limit" in spruce_hip.last_error()


def test_project_levels_validation_before_launch():
    lib = spruce_hip.lib()
    fake = ctypes.c_void_p(1 << 20)
    levels = (ctypes.c_void_p * 2)(fake, fake)
    nodes = (ctypes.c_int64 * 2)(4, 2)
    cases = [((levels, nodes, 0, 1, 8, 128, 0, fake, 128, fake, 0, None), "between 1 and 32 levels"),
             ((levels, nodes, 33, 1, 8, 128, 0, fake, 128, fake, 0, None), "between 1 and 32 levels"),
             ((levels, nodes, 2, 1, 8, 126, 0, fake, 128, fake, 0, None), "multiples of 4"),
             ((levels, nodes, 2, 1, 8, 128, 9, fake, 128, fake, 0, None), "unsupported dtype"),
             (((ctypes.c_void_p * 2)(fake, None), nodes, 2, 1, 8, 128, 0, fake, 128, fake, 0, None), "level 1"),
             (((ctypes.c_void_p * 2)(fake, ctypes.c_void_p((1 << 20) + 2)), nodes, 2, 1, 8, 128, 0, fake, 128,
               fake, 0, None), "not 8-byte aligned"),
             ((levels, nodes, 2, 1, 8, 128, 0, fake, 128, fake, 3, None), "unknown output layout")]
    for args, message in cases:
        assert lib.spruce_gate_project_levels(*args) == -1, message
        assert message in spruce_hip.last_error(), (message, spruce_hip.last_error())


def test_attention_mask_validation_before_launch():
    lib = spruce_hip.lib()
    fake = ctypes.c_void_p(1 << 20)
    st = _strides(0, 0, 128, 1)

    def call(amask=fake, ams=(0, 0, 64, 1), Hm=1, Tq=64, Tk=64, code=2, scale=0.1):
        return lib.spruce_sparse_prefill_index_amask(
            fake, st, fake, st, fake, st, fake, _strides(0, 0, 1, 1), 1,
            amask, _strides(*ams), Hm, Tq, Tk, code, 1, 4, 2, 64, 128, scale, 0, 0,
            fake, _strides(0, 128, 512, 1), None)

    cases = [(dict(amask=None), "non-null"),
             (dict(Hm=2), "1 or Hq"),
             (dict(Tq=63), "must cover"),
             (dict(Tk=32), "must cover"),
             (dict(ams=(0, 0, 64, 2)), "contiguous last dimension"),
             (dict(ams=(-64, 0, 64, 1)), "negative"),
             (dict(code=7), "mask dtype"),
             (dict(scale=0.0), "finite nonzero scale"),
             (dict(scale=float("inf")), "finite nonzero scale")]
    for kwargs, message in cases:
        assert call(**kwargs) == -1, kwargs
        assert message in spruce_hip.last_error(), (kwargs, spruce_hip.last_error())


def test_summary_table_dtype_validation_before_launch():
    # The summary table is float32 or a copy in the 16-bit input dtype.
    lib = spruce_hip.lib()
    fake = ctypes.c_void_p(1 << 20)
    st = _strides(0, 0, 128, 1)

    def call(dtype, sum_dtype):
        return lib.spruce_sparse_prefill_index_summaries(
            fake, st, fake, st, fake, st, fake, _strides(0, 0, 1, 1), 1,
            fake, _strides(0, 0, 1, 1), 1, fake, fake, fake, sum_dtype, 3, 1,
            1, 4, 2, 64, 128, 0.1, dtype, 0, fake, _strides(0, 128, 512, 1), None)

    for dtype, sum_dtype in ((0, 1), (1, 0), (2, 0), (0, 7)):
        assert call(dtype, sum_dtype) == -1, (dtype, sum_dtype)
        assert "float32 or the 16-bit input dtype" in spruce_hip.last_error(), spruce_hip.last_error()


def test_fused_selector_support_and_validation_before_launch():
    lib = spruce_hip.lib()
    bf16, f32 = 0, 2
    assert lib.spruce_select_flat_supported(28, 4, 65536, 128, bf16, 128) == 1
    assert lib.spruce_select_flat_supported(28, 4, 65537, 128, bf16, 128) == 0     # 1025 key blocks
    assert lib.spruce_select_flat_supported(36, 4, 1000, 128, bf16, 128) == 0      # 9 query heads per KV head
    assert lib.spruce_select_flat_supported(28, 4, 1000, 64, bf16, 128) == 0
    assert lib.spruce_select_flat_supported(28, 4, 1000, 128, f32, 128) == 0
    assert lib.spruce_select_flat_supported(28, 4, 1000, 128, bf16, 64) == 0
    assert lib.spruce_select_flat_workspace_bytes(1, 4, 65536, 128) == 4 * 2 * 128 * 1024 * 4
    fake = ctypes.c_void_p(1 << 20)
    qs, ks = _strides(0, 128 * 1000, 128, 1), _strides(0, 128 * 1000, 128, 1)
    need = lib.spruce_select_flat_workspace_bytes(1, 4, 1000, 128)

    def call(Hq=28, T=1000, D=128, dtype=bf16, P=128, top_k=32, ws_bytes=need, ws=fake, qs=qs, out=fake):
        return lib.spruce_select_flat(fake, qs, fake, ks, 1, Hq, 4, T, D, dtype, fake, fake, P, 11.3, top_k,
                                      ws, ws_bytes, out, None)
    cases = [(dict(D=64), "head_dim 128"), (dict(dtype=f32), "head_dim 128"), (dict(Hq=36), "head_dim 128"),
             (dict(T=65537), "head_dim 128"), (dict(P=64), "head_dim 128"), (dict(top_k=0), "top_k"),
             (dict(ws_bytes=need - 4), "workspace too small"), (dict(ws=ctypes.c_void_p((1 << 20) + 4)), "aligned"),
             (dict(qs=_strides(0, 128 * 1000, 100, 1)), "16-byte aligned"), (dict(out=None), "non-null"),
             (dict(Hq=30), "invalid shape")]
    for kwargs, message in cases:
        assert call(**kwargs) == -1, kwargs
        assert message in spruce_hip.last_error(), (kwargs, spruce_hip.last_error())


def test_pooled_projection_validation_before_launch():
    lib = spruce_hip.lib()
    fake = ctypes.c_void_p(1 << 20)
    qs, ks = _strides(0, 128, 3584, 1), _strides(0, 128, 512, 1)

    def call(Hq=28, D=128, dtype=0, P=128, qs=qs, out=fake, T=1000):
        return lib.spruce_selector_pool_project(fake, qs, fake, ks, 1, Hq, 4, T, D, dtype, fake, fake, P, out,
                                                fake, None)
    cases = [(dict(D=64), "head_dim 128"), (dict(dtype=2), "16-bit"), (dict(Hq=36), "at most 8"),
             (dict(P=64), "projection dim 128"), (dict(qs=_strides(0, 128, 100, 1)), "16-byte aligned"),
             (dict(out=None), "non-null"), (dict(Hq=30), "invalid shape"),
             (dict(qs=_strides(0, 128, 1 << 22, 1), T=1 << 10), "2^31")]
    for kwargs, message in cases:
        assert call(**kwargs) == -1, kwargs
        assert message in spruce_hip.last_error(), (kwargs, spruce_hip.last_error())


def test_proto_pool_qk_validation_before_launch():
    lib = spruce_hip.lib()
    fake = ctypes.c_void_p(1 << 20)
    qs, ks = _strides(0, 128, 3584, 1), _strides(0, 128, 512, 1)

    def call(Hq=28, D=128, dtype=0, block=64, P=8, qs=qs, out=fake):
        return lib.spruce_proto_pool_qk(fake, qs, fake, ks, 1, Hq, 4, 1000, D, block, P, dtype, out, fake, None)
    cases = [(dict(dtype=2), "16-bit"), (dict(D=12), "multiple of 8"), (dict(Hq=36), "at most 8"),
             (dict(block=65), "block must be"), (dict(P=66), "P must be"), (dict(out=None), "non-null"),
             (dict(qs=_strides(0, 128, 100, 1)), "16-byte aligned"), (dict(Hq=30), "not divisible")]
    for kwargs, message in cases:
        assert call(**kwargs) == -1, kwargs
        assert message in spruce_hip.last_error(), (kwargs, spruce_hip.last_error())
