"""Sparse-prefill benchmark on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu] [--no-csr128k] [--no-extra]

One step = one block-sparse causal GQA prefill of a Qwen2-7B-shaped attention
layer (the headline configuration cfg2: T=32768, 28 query / 4 KV heads, d=128, bf16 Q/K/V ~
N(0,1) with RoPE theta=1e6, block mask of sink + local-4 + stable top-k at
~10% causal density), launched through the C ABI
(spruce_sparse_prefill_mask) with inputs already resident in HBM.

Printed: one JSON line with the headline metric (effective TFLOP/s over the
computed blocks, 4*64*64*128 FLOP per (query head, selected block)), ms per
step, the live roofline of the kernel (HIP events on the launch stream) and a
CPU baseline (the float32 numpy oracle on a bounded sample of the same
workload).  The reference's small fp32 case (cfg1), the 128K direct-index CSR
configuration (cfg5) with its tree-route producer stage by stage, the selector
front end (cfg3, HBM-bound: GB/s) and teacher block-mass extraction (cfg4) are
timed the same way and reported under "configs".
"""
import argparse
import json
import os
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
for _p in (os.path.join(ROOT, "spruce-research_amd"), ROOT):
    if _p not in sys.path:
        sys.path.insert(0, _p)

PEAK_BF16_TFLOPS = 2500.0  # MI355X dense bf16 MFMA
PEAK_FP32_TFLOPS = 157.3   # MI355X fp32 (vector, with packed FP32)
PEAK_HBM_GBS = 8000.0
BLOCK_FLOPS = 4.0 * 64 * 64 * 128  # per (query head, selected 64-key block), d=128


def _time_launches(fn, steps, warmup):
    """Run fn warmup times, then time `steps` launches.

    Returns (wall ms per step bracketed by synchronize, list of per-launch
    kernel ms from HIP events recorded on the launch stream)."""
    import torch
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream()
    events = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
              for _ in range(steps)]
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for s, e in events:
        s.record(stream)
        fn()
        e.record(stream)
    torch.cuda.synchronize()
    wall_ms = (time.perf_counter() - t0) * 1e3 / steps
    return wall_ms, [s.elapsed_time(e) for s, e in events]


def _traffic(name):
    """HBM bytes per launch from the committed rocprofv3 PMC summary, if any."""
    path = os.path.join(ROOT, "profiles", "traffic.json")
    try:
        with open(path) as f:
            return json.load(f).get(name)
    except (OSError, ValueError):
        return None


def _cpu_model():
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    import platform
    return platform.processor() or "unknown"


def _numpy_threads():
    try:
        from threadpoolctl import threadpool_info
        return max((i.get("num_threads") or 0) for i in threadpool_info()) or None
    except Exception:
        return None


def _cpu_time(fn):
    """One untimed warm-up call, then the median of three timed calls (s)."""
    fn()
    ts = []
    for _ in range(3):
        t0 = time.perf_counter()
        fn()
        ts.append(time.perf_counter() - t0)
    return statistics.median(ts)


def cpu_baseline(q, k, v, mask_kv, sample_blocks):
    """Time the float32 numpy oracle on a sample of query blocks of cfg2."""
    import numpy as np

    import oracle.attention as ora
    threads = _numpy_threads()
    qn, kn, vn = (x.float().cpu().numpy() for x in (q, k, v))
    mk = mask_kv.cpu().numpy()
    ora.sparse_attention_mask(qn, kn, vn, mk, qblocks_subset=sample_blocks[:1])  # warm-up
    t0 = time.perf_counter()
    ora.sparse_attention_mask(qn, kn, vn, mk, qblocks_subset=sample_blocks)
    dt = time.perf_counter() - t0
    G = q.shape[1] // k.shape[1]
    sel = sum(int(mk[0, g, s, : s + 1].sum()) for g in range(mk.shape[1]) for s in sample_blocks)
    flops = sel * G * BLOCK_FLOPS
    return {
        "value": round(flops / dt / 1e12, 6),
        "unit": "TFLOP/s",
        "cores": threads or os.cpu_count(),
        "cpu_model": _cpu_model(),
        "kind": "port",
        "seconds": round(dt, 3),
        "sample": (f"oracle/attention.py float32 numpy, {len(sample_blocks)} of 512 query blocks "
                   f"x 4 KV heads x 7 query heads of cfg2, {sel * G} head-blocks"),
    }


def cpu_baseline_cfg1(q1, k1, v1, mask1, flops):
    """cfg1 on the host, the whole configuration: the float32 numpy oracle
    (oracle/attention.py, the reference's PyTorch path restated), median of 3."""
    import oracle.attention as ora
    qn, kn, vn, mn = (x.numpy() for x in (q1, k1, v1, mask1))
    dt = _cpu_time(lambda: ora.sparse_attention_mask(qn, kn, vn, mn))
    return {"value": round(flops / dt / 1e12, 6), "unit": "TFLOP/s", "ms": round(dt * 1e3, 2),
            "cores": _numpy_threads() or os.cpu_count(), "cpu_model": _cpu_model(), "kind": "port",
            "seconds": round(dt, 3),
            "sample": "whole cfg1 (8 query heads x 64 query blocks), float32 numpy, median of 3"}


def cpu_baseline_selector(q3, k3, Wq, Wk, top_k, nbytes):
    """cfg3 on the host: the reference's flat selector restated with float32
    torch ops (oracle/reference_cpu.py), the whole configuration."""
    import torch

    import oracle.reference_cpu as rc
    qc, kc = q3.cpu(), k3.cpu()
    dt = _cpu_time(lambda: rc.flat_select(qc, kc, Wq, Wk, top_k=top_k))
    return {"value": round(nbytes / dt / 1e9, 3), "unit": "GB/s", "cores": torch.get_num_threads(),
            "cpu_model": _cpu_model(), "kind": "port", "seconds": round(dt, 3),
            "sample": "whole cfg3 (group mean, block mean/max, projections, MaxSim, stable top-32), "
                      "float32 torch, median of 3"}


def cpu_baseline_teacher(q4, k4, scale, heads, flop_per_head):
    """cfg4 on the host: the reference's chunked_pool (float32 torch,
    oracle/reference_cpu.py) on a slice of query heads, plus the targets of
    the full mass tensor."""
    import torch

    import oracle.reference_cpu as rc
    qc, kc = q4.cpu(), k4.cpu()
    H = qc.shape[1]

    def run():
        mass = rc.chunked_pool(qc, kc, scale, heads=heads)
        rc.teacher_targets(mass, kc.shape[1], k=8)

    dt = _cpu_time(run)
    return {"value": round(flop_per_head * len(heads) / dt / 1e12, 6), "unit": "TFLOP/s",
            "cores": torch.get_num_threads(), "cpu_model": _cpu_model(), "kind": "port",
            "seconds": round(dt, 3),
            "sample": (f"chunked_pool on {len(heads)} of {H} query heads (all 256 query blocks) + "
                       "targets, float32 torch, median of 3; TFLOP/s over the sampled heads")}


def cpu_baseline_csr(q5, k5, v5, indptr, indices, kv_head, qblocks, G):
    """cfg5 on the host: the float32 numpy oracle (oracle/attention.py) on one
    KV head and a sample of its query blocks."""
    import numpy as np

    import oracle.attention as ora
    Qb = indptr.numel() // k5.shape[1]
    qs = q5[:, kv_head * G:(kv_head + 1) * G].float().cpu().numpy()
    ks = k5[:, kv_head:kv_head + 1].float().cpu().numpy()
    vs = v5[:, kv_head:kv_head + 1].float().cpu().numpy()
    ip = indptr[kv_head * Qb:(kv_head + 1) * Qb + 1]
    ip_n = (ip - ip[0]).numpy()
    ix_n = indices[int(ip[0]):int(ip[-1])].numpy()
    t0 = time.perf_counter()
    ora.sparse_attention_csr(qs, ks, vs, ip_n, ix_n, qblocks_subset=qblocks)
    dt = time.perf_counter() - t0
    blocks = sum(int(ip_n[r + 1] - ip_n[r]) for r in qblocks)
    return {"value": round(blocks * G * BLOCK_FLOPS / dt / 1e12, 6), "unit": "TFLOP/s",
            "cores": _numpy_threads() or os.cpu_count(), "cpu_model": _cpu_model(), "kind": "port",
            "seconds": round(dt, 3),
            "sample": (f"oracle/attention.py float32 numpy, KV head {kv_head} (7 query heads), "
                       f"{len(qblocks)} of {Qb} query blocks, {blocks} listed key blocks")}


def main():
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--seed", type=int, default=0)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--no-csr128k", action="store_true", help="skip the 128K CSR configuration")
    ap.add_argument("--no-extra", action="store_true", help="skip the selector (cfg3) and teacher (cfg4) legs")
    ap.add_argument("--calib-copy", action="store_true",
                    help="after timing, run one plain 512 MiB device copy (PMC byte calibration)")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU's share of the layer; multi-GPU runs are not part of "
              "this build (the layer shards by KV head, each GPU owning whole KV heads, with no exchange)",
              file=sys.stderr)
        sys.exit(2)

    import torch

    from kernels.block_mask import block_sparse_prefill
    from kernels.direct_index import csr_row_order, direct_index_sparse_csr
    from spruce_hip import workloads

    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)

    # ---- cfg2: Qwen2-7B layer, T=32768, block mask at ~10% density
    T, Hq, Hkv, D = 32768, 28, 4, 128
    q, k, v = workloads.qkv(args.seed, T, Hq, Hkv, D, torch.bfloat16, use_rope=True,
                            layout="bthd", device="cuda")
    mask, density = workloads.cfg2_mask(args.seed)
    mask_d = mask.to(dev)
    selected = int(mask[:, ::Hq // Hkv].sum())
    flops = selected * (Hq // Hkv) * BLOCK_FLOPS
    scale = D ** -0.5
    fn = lambda: block_sparse_prefill(q, k, v, mask_d, scale)  # noqa: E731
    wall_ms, kern_ms = _time_launches(fn, args.steps, args.warmup)
    kmean = statistics.fmean(kern_ms)
    kmed = statistics.median(kern_ms)
    achieved = flops / (kmean * 1e-3) / 1e12

    configs = {
        "cfg2_32k_block_mask": {
            "ms_median": round(kmed, 4), "ms_min": round(min(kern_ms), 4),
            "ms_max": round(max(kern_ms), 4),
            "tflops": round(flops / (kmed * 1e-3) / 1e12, 2),
            "frac_bf16_peak": round(flops / (kmed * 1e-3) / 1e12 / PEAK_BF16_TFLOPS, 4),
            "density": round(density, 5), "selected_kv_blocks": selected, "flop": flops,
        }
    }

    # ---- cfg1: the reference's CPU-runnable case (T=4096, 8 query / 2 KV
    # heads, fp32 N(0,1) Q/K/V, top-16 + sink + diagonal per KV head, bool
    # mask [1, 8, 64, 64]); fp32 inputs are rounded to bf16 for the matrix cores.
    q1, k1, v1 = workloads.qkv(args.seed, 4096, 8, 2, D, torch.float32, use_rope=False)
    mask1 = workloads.cfg1_mask(args.seed)
    q1d, k1d, v1d, m1d = (x.to(dev) for x in (q1, k1, v1, mask1))
    sel1 = int(mask1.sum())
    flops1 = sel1 * BLOCK_FLOPS
    fn1 = lambda: block_sparse_prefill(q1d, k1d, v1d, m1d, scale)  # noqa: E731
    _, k1ms = _time_launches(fn1, max(10, args.steps // 2), max(3, args.warmup // 2))
    m1 = statistics.median(k1ms)
    configs["cfg1_4k_block_mask_fp32"] = {
        "ms_median": round(m1, 4), "ms_min": round(min(k1ms), 4), "ms_max": round(max(k1ms), 4),
        "tflops": round(flops1 / (m1 * 1e-3) / 1e12, 2),
        "frac_bf16_peak": round(flops1 / (m1 * 1e-3) / 1e12 / PEAK_BF16_TFLOPS, 4),
        "selected_head_blocks": sel1, "flop": flops1, "input_dtype": "fp32",
        "note": "128 (KV head, query block) rows split into 2 four-wave parts: 256 workgroups, "
                "one per CU, each over a few blocks, so this small case is launch- and "
                "latency-bound",
    }
    if not args.no_cpu:
        configs["cfg1_4k_block_mask_fp32"]["cpu_baseline"] = cpu_baseline_cfg1(q1, k1, v1, mask1, flops1)
    del q1d, k1d, v1d, m1d

    # ---- cfg5: T=131072 direct-index CSR with log-normal row densities
    if not args.no_csr128k:
        T5 = 131072
        q5, k5, v5 = workloads.qkv(args.seed, T5, Hq, Hkv, D, torch.bfloat16, use_rope=True,
                                   layout="bthd", device="cuda")
        indptr, indices = workloads.cfg5_csr(args.seed)
        ip, ix = indptr.to(dev), indices.to(dev)
        order = csr_row_order(ip, Hkv)
        nnz = int(indices.numel())
        flops5 = nnz * (Hq // Hkv) * BLOCK_FLOPS
        fn5 = lambda: direct_index_sparse_csr(q5, k5, v5, ip, ix, scale, row_order=order)  # noqa: E731
        _, k5ms = _time_launches(fn5, max(5, args.steps // 5), max(2, args.warmup // 5))
        m5 = statistics.median(k5ms)
        counts = (indptr[1:] - indptr[:-1]).float()
        configs["cfg5_128k_csr"] = {
            "ms_median": round(m5, 4), "ms_min": round(min(k5ms), 4), "ms_max": round(max(k5ms), 4),
            "tflops": round(flops5 / (m5 * 1e-3) / 1e12, 2),
            "frac_bf16_peak": round(flops5 / (m5 * 1e-3) / 1e12 / PEAK_BF16_TFLOPS, 4),
            "nnz_kv_blocks": nnz, "flop": flops5,
            "row_blocks_mean": round(float(counts.mean()), 2), "row_blocks_max": int(counts.max()),
        }
        if not args.no_cpu:
            configs["cfg5_128k_csr"]["cpu_baseline"] = cpu_baseline_csr(
                q5, k5, v5, indptr, indices, 0, list(range(0, 2048, 4)), Hq // Hkv)
        # Tree route producer at the cfg5 grid (deployed settings of the
        # reference's export script: radix 2, beam 16, local window 1,
        # k_selected = beam + 2): prototype features of Q and K, the key tree,
        # projections, beam traversal and packing into selected_blocks.  The
        # whole route is timed, then each stage on its own (inputs from one
        # untimed run), each against the roofline of its algorithmic work.
        if not args.no_extra:
            import math
            from interfaces.packing import selected_ids_to_blocks
            from selector.gate import FlatGate
            from selector.traversal import traverse_projected
            from selector.tree import build_key_tree
            from teacher.chunked_extract import proto_pool_qk
            kb5, beam = T5 // 64, 16
            gate = FlatGate(1, D, proj_dim=D).to(dev).eval()
            div = math.sqrt(gate.proj_dim)

            def features():
                return proto_pool_qk(q5, k5, 64, 8)

            def project(qf, levels):
                return gate.project_queries(qf), gate.project_key_levels([lvl.features for lvl in levels],
                                                                          interleaved=True)

            def route():
                qf, kf = features()
                levels = build_key_tree(kf, radix=2)
                qp, kp = project(qf, levels)
                ids = traverse_projected(qp, kp, kb5, beam, 2, div)
                return selected_ids_to_blocks(ids, beam + 2, local_window=1, key_blocks=kb5)

            rsteps, rwarm = max(5, args.steps // 5), max(2, args.warmup // 5)
            _, krms = _time_launches(route, rsteps, rwarm)
            qf, kf = features()
            levels = build_key_tree(kf, radix=2)
            qp, kp = project(qf, levels)
            ids = traverse_projected(qp, kp, kb5, beam, 2, div)
            stage_fns = {
                "features": features,
                "tree": lambda: build_key_tree(kf, radix=2),
                "project": lambda: project(qf, levels),
                "traverse": lambda: traverse_projected(qp, kp, kb5, beam, 2, div),
                "pack": lambda: selected_ids_to_blocks(ids, beam + 2, local_window=1, key_blocks=kb5),
            }
            work = workloads.tree_route_work(T5, Hq, Hkv, D, P=8, proj=D, beam=beam, radix=2,
                                             k_selected=beam + 2)
            stages, floor_ms = {}, 0.0
            for name, sfn in stage_fns.items():
                _, sms = _time_launches(sfn, rsteps, rwarm)
                msd = statistics.median(sms)
                w = work[name]
                t_hbm = w["bytes"] / (PEAK_HBM_GBS * 1e9) * 1e3
                t_fp32 = w["flop"] / (PEAK_FP32_TFLOPS * 1e12) * 1e3
                bound = "fp32" if t_fp32 > t_hbm else "hbm"
                floor = max(t_hbm, t_fp32)
                floor_ms += floor
                stages[name] = {"ms_median": round(msd, 4), "bytes": w["bytes"], "flop": w["flop"],
                                "bound": bound, "floor_ms": round(floor, 4),
                                "frac": round(floor / msd, 4)}
                if bound == "fp32":
                    stages[name]["tflops"] = round(w["flop"] / (msd * 1e-3) / 1e12, 2)
                else:
                    stages[name]["gbps"] = round(w["bytes"] / (msd * 1e-3) / 1e9, 1)
            stages["traverse"]["candidates_per_row"] = work["traverse"]["candidates_per_row"]
            mr = statistics.median(krms)
            configs["cfg5_tree_route"] = {
                "ms_median": round(mr, 4), "ms_min": round(min(krms), 4), "ms_max": round(max(krms), 4),
                "floor_ms": round(floor_ms, 4), "frac": round(floor_ms / mr, 4),
                "key_blocks": kb5, "kv_groups": Hkv, "prototypes": 8, "proj_dim": D, "beam": beam,
                "radix": 2, "k_selected": beam + 2,
                "stages": stages,
                "note": ("floor = sum over stages of max(bytes / 8 TB/s, flop / 157.3 TFLOP/s fp32); "
                         "traverse is the dominant kernel (tree_traverse_kernel, fp32 VALU dot products; "
                         "157.3 TFLOP/s assumes packed FP32, which this build does not emit, so 78.6 is "
                         "its VALU ceiling)"),
            }
            del qf, kf, levels, qp, kp, ids
        del q5, k5, v5

    # ---- capture pass: dense causal cfg2 layer that also emits the selector
    # features (group-averaged Q, key prototypes; the Q prototypes pooled by
    # one small launch), against the same work done in separate passes.
    if not args.no_extra:
        from teacher.chunked_extract import causal_prefill_features, proto_pool_qk
        fnc = lambda: causal_prefill_features(q, k, v, scale, 8)  # noqa: E731
        fnu = lambda: (causal_prefill_features(q, k, v, scale, capture=False),  # noqa: E731
                       proto_pool_qk(q, k, 64, 8))
        _, kums = _time_launches(fnu, max(5, args.steps // 5), max(2, args.warmup // 5))
        _, kcms = _time_launches(fnc, max(5, args.steps // 5), max(2, args.warmup // 5))
        mc, mu = statistics.median(kcms), statistics.median(kums)
        qbk = T // 64
        flc = qbk * (qbk + 1) // 2 * Hq * BLOCK_FLOPS
        configs["cfg2_capture_32k"] = {
            "ms_median": round(mc, 4), "ms_min": round(min(kcms), 4), "ms_max": round(max(kcms), 4),
            "tflops": round(flc / (mc * 1e-3) / 1e12, 2),
            "frac_bf16_peak": round(flc / (mc * 1e-3) / 1e12 / PEAK_BF16_TFLOPS, 4),
            "flop": flc, "prototypes": 8,
            "separate_passes_ms_median": round(mu, 4),
            "stages": "dense causal attention + group-averaged Q + key prototypes in one pass, "
                      "then Q prototypes pooled from the grouped tokens",
        }

    # ---- residual summaries on the cfg2 selection: the frontier nodes of
    # every row, the layer's K/V summary table (one prototype per node) and
    # the direct-index kernel with the summary keys appended, against the
    # same kernel without them.  FLOPs count the exact keys plus the listed
    # summary keys.
    if not args.no_extra:
        from interfaces.residual_summaries import build_residual_summary_nodes, build_residual_tree_layout
        from kernels.direct_index import direct_index_sparse_prefill, direct_index_sparse_summaries
        from sparse.summaries import build_kv_summary_table
        sel_r = workloads.mask_to_selected_blocks(mask[:, ::Hq // Hkv])[:, None].to(dev)
        idx_r = sel_r[:, 0].contiguous()
        nodes_r = build_residual_summary_nodes(sel_r, validate_selected=False)[:, 0].to(torch.int32).contiguous()
        lay_r = build_residual_tree_layout(idx_r.shape[2])

        def fnr():
            table = build_kv_summary_table(k, v, lay_r, block_size=64, prototypes=1)
            return direct_index_sparse_summaries(q, k, v, idx_r, nodes_r, table, scale=scale)

        fnp_ = lambda: direct_index_sparse_prefill(q, k, v, idx_r, scale=scale)  # noqa: E731
        _, krms_ = _time_launches(fnr, max(5, args.steps // 5), max(2, args.warmup // 5))
        _, kpms_ = _time_launches(fnp_, max(5, args.steps // 5), max(2, args.warmup // 5))
        mr_, mp_ = statistics.median(krms_), statistics.median(kpms_)
        entries = int((nodes_r >= 0).sum())
        flr = flops + entries * (Hq // Hkv) * BLOCK_FLOPS // 64
        configs["cfg2_residual_summaries_32k"] = {
            "ms_median": round(mr_, 4), "ms_min": round(min(krms_), 4), "ms_max": round(max(krms_), 4),
            "tflops": round(flr / (mr_ * 1e-3) / 1e12, 2),
            "frac_bf16_peak": round(flr / (mr_ * 1e-3) / 1e12 / PEAK_BF16_TFLOPS, 4),
            "flop": flr, "summary_keys": entries, "prototypes": 1,
            "without_summaries_ms_median": round(mp_, 4),
            "stages": "K/V summary table of the layer, then direct-index attention over the listed "
                      "blocks and the row's frontier-node summary keys in one softmax",
        }

    # ---- cfg3: selector front end, T=65536 (1024 key blocks), top-32
    if not args.no_extra:
        from selector.select import select_blocks
        T3 = 65536
        q3, k3, v3 = workloads.qkv(args.seed, T3, Hq, Hkv, D, torch.bfloat16, use_rope=False,
                                   layout="bthd", device="cuda")
        Wq, Wk = (w.to(dev) for w in workloads.cfg3_gate_weights(args.seed))
        fn3 = lambda: select_blocks(q3, k3, Wq, Wk, top_k=32)  # noqa: E731
        _, k3ms = _time_launches(fn3, max(10, args.steps // 2), max(3, args.warmup // 2))
        m3 = statistics.median(k3ms)
        by3 = workloads.selector_bytes(T3, Hq, Hkv, D, 32)
        configs["cfg3_selector_64k"] = {
            "ms_median": round(m3, 4), "ms_min": round(min(k3ms), 4), "ms_max": round(max(k3ms), 4),
            "gbps": round(by3 / (m3 * 1e-3) / 1e9, 1),
            "frac_hbm_peak": round(by3 / (m3 * 1e-3) / 1e9 / PEAK_HBM_GBS, 4),
            "compulsory_bytes": by3, "top_k": 32,
            "stages": "pool (Q group+block mean, K mean/max) and project, one launch -> MaxSim scores -> causal top-k",
        }
        if not args.no_cpu:
            configs["cfg3_selector_64k"]["cpu_baseline"] = cpu_baseline_selector(
                q3, k3, Wq.cpu(), Wk.cpu(), 32, by3)

        # Selector prototype features of the reference's capture hook: Q
        # group-averaged and pooled to mean + 7 outliers per block, K likewise.
        from teacher.chunked_extract import proto_pool_qk
        fnp = lambda: proto_pool_qk(q3, k3, 64, 8)  # noqa: E731
        _, kpms = _time_launches(fnp, max(10, args.steps // 2), max(3, args.warmup // 2))
        mp = statistics.median(kpms)
        byp = (Hq + Hkv) * T3 * D * 2 + 2 * Hkv * (T3 // 64) * 8 * D * 2
        configs["cfg3_proto_features_64k"] = {
            "ms_median": round(mp, 4), "ms_min": round(min(kpms), 4), "ms_max": round(max(kpms), 4),
            "gbps": round(byp / (mp * 1e-3) / 1e9, 1),
            "frac_hbm_peak": round(byp / (mp * 1e-3) / 1e9 / PEAK_HBM_GBS, 4),
            "compulsory_bytes": byp, "prototypes": 8,
        }

        # Residual-tree K/V summary table (4 positional prototypes per node).
        from interfaces.residual_summaries import build_residual_tree_layout
        from sparse.summaries import build_kv_summary_table
        k3h, v3h = k3.contiguous(), v3.contiguous()
        lay = build_residual_tree_layout(T3 // 64)
        fns = lambda: build_kv_summary_table(k3h, v3h, lay, block_size=64, prototypes=4)  # noqa: E731
        _, ksms = _time_launches(fns, max(10, args.steps // 2), max(3, args.warmup // 2))
        ms_ = statistics.median(ksms)
        bys = 2 * Hkv * T3 * D * 2 + 2 * Hkv * lay.num_nodes * 4 * D * 4 + 2 * lay.num_nodes * 4 * 4
        configs["cfg3_kv_summaries_64k"] = {
            "ms_median": round(ms_, 4), "ms_min": round(min(ksms), 4), "ms_max": round(max(ksms), 4),
            "gbps": round(bys / (ms_ * 1e-3) / 1e9, 1),
            "frac_hbm_peak": round(bys / (ms_ * 1e-3) / 1e9 / PEAK_HBM_GBS, 4),
            "compulsory_bytes": bys, "nodes": lay.num_nodes, "prototypes": 4,
            "stages": "dyadic table of K and V (one read), upper table levels, one entry per node prototype",
            "note": "the host call's torch allocations are inside the timed region; the token-range "
                    "table is built once per layout and cached",
        }
        del q3, k3, v3, k3h, v3h

    # ---- route packing at the cfg5 grid: 4 KV heads x 2048 query blocks,
    # 96 traversal candidates per row into 64-wide selected_blocks rows.
    if not args.no_extra:
        from interfaces.packing import selected_ids_to_blocks
        gen = torch.Generator(device=dev).manual_seed(args.seed)
        ids6 = torch.randint(0, 2048, (1, Hkv, 2048, 96), generator=gen, device=dev, dtype=torch.int64)
        fn6 = lambda: selected_ids_to_blocks(ids6, 64, 1, None, 1)  # noqa: E731
        _, k6ms = _time_launches(fn6, max(10, args.steps // 2), max(3, args.warmup // 2))
        m6 = statistics.median(k6ms)
        by6 = ids6.numel() * 8 + Hkv * 2048 * 64 * 4
        configs["cfg5_route_packing"] = {
            "ms_median": round(m6, 4), "ms_min": round(min(k6ms), 4), "ms_max": round(max(k6ms), 4),
            "gbps": round(by6 / (m6 * 1e-3) / 1e9, 1),
            "frac_hbm_peak": round(by6 / (m6 * 1e-3) / 1e9 / PEAK_HBM_GBS, 4),
            "compulsory_bytes": by6, "rows": Hkv * 2048, "candidates": 96, "k_selected": 64,
        }
        del ids6

    # ---- cfg4: teacher block mass + targets, T=16384 (256 blocks)
    if not args.no_extra:
        from teacher.chunked_extract import chunked_pool
        from teacher.targets import teacher_targets
        T4 = 16384
        q4, k4, _ = workloads.qkv(args.seed, T4, Hq, Hkv, D, torch.bfloat16, use_rope=True,
                                  layout="bthd", device="cuda")
        fn4 = lambda: teacher_targets(chunked_pool(q4, k4, scale), Hkv, k=8)  # noqa: E731
        _, k4ms = _time_launches(fn4, max(10, args.steps // 2), max(3, args.warmup // 2))
        m4 = statistics.median(k4ms)
        fl4 = workloads.teacher_flops(T4, Hq)
        configs["cfg4_teacher_16k"] = {
            "ms_median": round(m4, 4), "ms_min": round(min(k4ms), 4), "ms_max": round(max(k4ms), 4),
            "tflops": round(fl4 / (m4 * 1e-3) / 1e12, 2),
            "frac_bf16_peak": round(fl4 / (m4 * 1e-3) / 1e12 / PEAK_BF16_TFLOPS, 4),
            "flop": fl4, "top_k": 8,
            "note": "algorithmic FLOP = QK^T once over causal blocks (the single-pass kernel computes it once)",
        }
        if not args.no_cpu:
            configs["cfg4_teacher_16k"]["cpu_baseline"] = cpu_baseline_teacher(
                q4, k4, scale, list(range(0, Hq, 4)), fl4 / Hq)
        del q4, k4

    if args.calib_copy:
        # A plain copy of known size: reads and writes exactly 512 MiB.  Its
        # FETCH_SIZE / WRITE_SIZE readings calibrate the PMC byte counters.
        src = torch.empty(256 * 1024 * 1024, dtype=torch.bfloat16, device=dev).fill_(1)
        dst = torch.empty_like(src)
        torch.cuda.synchronize()
        dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst

    cpu = None
    if not args.no_cpu:
        sample = list(range(512))
        cpu = cpu_baseline(q, k, v, mask[:, ::Hq // Hkv], sample)

    result = {
        "metric": "sparse-prefill attn ms + effective TFLOP/s, Qwen2-7B layer @32K/128K, 1 GPU",
        "value": round(flops / (wall_ms * 1e-3) / 1e12, 3),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(wall_ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded N(0,1) Q/K/V with RoPE, generated on the GPU; seeded block mask)",
        "config": {
            "workload": "cfg2: Qwen2-7B attention layer, block-sparse causal GQA prefill, block mask",
            "seq_len": T, "query_heads": Hq, "kv_heads": Hkv, "head_dim": D, "block": 64,
            "density": round(density, 5), "batch": 1, "parallelism": "none (1 GPU)",
        },
        "roofline": {
            "bound": "mfma",
            "achieved": round(achieved, 2),
            "peak": PEAK_BF16_TFLOPS,
            "unit": "TFLOP/s",
            "frac": round(achieved / PEAK_BF16_TFLOPS, 4),
            "traffic": _traffic("cfg2_32k_block_mask"),
            "kernel": "sparse_prefill_kernel<128, 8, InBF16, false, 2, false, false, true> (block mask, producer wave)",
            "kernel_ms_mean": round(kmean, 4),
        },
        "cpu_baseline": cpu,
        "configs": configs,
    }
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
