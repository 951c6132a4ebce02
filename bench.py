#!/usr/bin/env python
"""Sparse decode attention benchmark on one MI355X.

Metric: sparse decode attention us/layer + HBM GB/s (% of
peak) at N=32K, B=4, c=0.15 -- configuration C2: Llama-3.2-1B heads
(32 Q / 8 KV, D=64), B=4, N=32768, k=ceil(0.15*N)=4916, fp16 K/V cache
[B, 8, N, 64], fp32 softmax.

A step is one call of the fused C-ABI entry point ``dcr_sparse_decode``
(score pass with u_Q and the level-1 histogram -> top-k select -> gather +
attention with the merge in its last workgroups: three launches) for one
layer, inputs resident in HBM.  Steps rotate over ``--layers`` independent
layer buffers (> 256 MB of K/V in total) so the 256 MB Infinity Cache is cold
for every step's score pass, as the reference measured one layer after
another.

Timing follows the reference's protocol (README.md:25-26: warm-up, then 3
sessions in randomized order): after the warm-up, each session times the
sparse path and the dense comparators (this build's dense HIP kernel, torch's
fused SDPA, the reference's eager dense branch) in a freshly shuffled order;
``value`` is the median over sessions of the sparse path's mean us per layer
(lower is better).  Per-kernel times come from HIP events attached to every
launch (hipExtLaunchKernelGGL start/stop events: the dispatch packet's own
begin and end timestamps) on the stream the kernels run on, in a further pass
over the same steps.  The line also carries the C3 end-to-end decode step
("e2e") and the CPU baseline: the reference's CPU path (its M1 torch calls,
restated in oracle/torch_twin.py) on the host's cores, with the C restatement
beside it.

Output: one JSON line (rank 0).
"""
from __future__ import annotations

import argparse
import json
import math
import os
import platform
import random
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
for _p in (ROOT, os.path.join(ROOT, "dcr-attention_v3_amd")):
    if _p not in sys.path:
        sys.path.insert(0, _p)

HBM_PEAK_GBPS = 8000.0  # MI355X HBM3E spec sheet


def parse_args():
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=50)
    ap.add_argument("--config", default="C2")
    ap.add_argument("--layers", type=int, default=6, help="rotating layer buffers (cold MALL)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-comparators", action="store_true")
    ap.add_argument("--configs", action="store_true",
                    help="also time the op at C1, C4a-c and C5 (B=1) against the dense kernel")
    ap.add_argument("--sessions", type=int, default=3,
                    help="timed sessions, each over every variant in a shuffled order")
    ap.add_argument("--seed", type=int, default=0, help="seed of the session orders")
    ap.add_argument("--no-e2e", action="store_true",
                    help="skip the end-to-end decode-step comparison (C3: 16-layer "
                         "Llama-3.2-1B shapes, B=4, 32K cache), reported as \"e2e\"")
    ap.add_argument("--e2e-steps", type=int, default=20)
    ap.add_argument("--rank-local", action="store_true",
                    help="only time the rank-local window attention (decode and prefill shapes) "
                         "and print its JSON object")
    ap.add_argument("--cpu-seconds", type=float, default=10.0,
                    help="host time spent on each CPU baseline's sample")
    ap.add_argument("--sparse-path", choices=("auto", "classic", "fused", "union"), default="auto",
                    help="auto: the library's choice (default; currently classic); classic: score, "
                         "select, index-list attention; fused: the whole step in one launch where the "
                         "shape allows it; union: union-gather attention")
    ap.add_argument("--score-form", choices=("auto", "valu"), default="auto",
                    help="score pass form: auto (MFMA chain where it fits) or valu (always VALU)")
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="only run a 256 MiB device-to-device copy 5 times (the reference "
                         "workload for scaling rocprofv3 FETCH_SIZE / WRITE_SIZE counters)")
    return ap.parse_args()


COPY_BYTES = 256 << 20


def calibrate_copy():
    """A plain copy of known size: rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE on
    this run give the counter's reading for COPY_BYTES read and written."""
    import torch
    src = torch.empty(COPY_BYTES, dtype=torch.uint8, device="cuda").random_(0, 255)
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    for _ in range(5):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"copy_bytes": COPY_BYTES, "copies": 5}), flush=True)


def load_traffic(config_name):
    """HBM bytes per launch per kernel, measured with rocprofv3 --pmc
    (FETCH_SIZE and WRITE_SIZE passes over this script, each scaled by the
    copy calibration) and committed as profiles/hbm_traffic_<config>.txt.
    Returns {kernel: bytes} or {} when no measurement is committed."""
    path = os.path.join(ROOT, "profiles", f"hbm_traffic_{config_name}.txt")
    out = {}
    if not os.path.exists(path):
        return out
    for line in open(path):
        f = line.split()
        if len(f) >= 2 and f[0] == "TRAFFIC":
            out[f[1]] = int(f[-1])
    return out


def env_stamp(torch):
    p = torch.cuda.get_device_properties(0)
    return {
        "device": p.name, "gcn_arch": getattr(p, "gcnArchName", ""),
        "cus": p.multi_processor_count, "torch": torch.__version__,
        "hip": getattr(torch.version, "hip", None), "host": platform.node(),
        "host_cpus": len(os.sched_getaffinity(0)),
    }


def main():
    args = parse_args()
    if args.calibrate_copy:
        calibrate_copy()
        return
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU only (--gpus {args.gpus} requested); "
              "the sparse decode path is per-GPU work and is not sharded here.", file=sys.stderr)
        sys.exit(2)

    import torch
    from dcr_attention_amd import _lib
    from dcr_attention_amd.synthetic import CONFIGS, make_qkv

    if args.rank_local:
        assert torch.cuda.is_available(), "bench.py needs a HIP device"
        print(json.dumps({"rank_local": rank_local_bench(torch, cpu=not args.no_cpu_baseline),
                          "env": env_stamp(torch)}), flush=True)
        return

    assert torch.cuda.is_available(), "bench.py needs a HIP device"
    cfg = CONFIGS[args.config]
    B, H, Hkv, N, D, k = cfg.B, cfg.H, cfg.Hkv, cfg.N, cfg.D, cfg.k
    dt = cfg.dtype
    esz = torch.tensor([], dtype=dt).element_size()
    dev = torch.device("cuda:0")
    lib = _lib.load()

    print(f"[bench] {cfg.name}: B={B} H={H} Hkv={Hkv} N={N} D={D} k={k} {dt}, "
          f"{args.layers} layers", file=sys.stderr, flush=True)
    layers = [make_qkv(B, H, Hkv, N, D, dt, seed=l, device="cuda", n_sinks=cfg.n_sinks,
                       sink_scale=cfg.sink_scale, n_outlier=cfg.n_outlier,
                       outlier_scale=cfg.outlier_scale) for l in range(args.layers)]
    ws_bytes = lib.dcr_sparse_decode_workspace_bytes(B, H, Hkv, N, D, k, _lib.DTYPE_CODE[dt])
    ws = _lib.workspace(ws_bytes, dev)
    out = torch.empty(B, H, D, dtype=dt, device=dev)
    code = _lib.DTYPE_CODE[dt]
    stream = torch.cuda.current_stream().cuda_stream
    ptrs = [(q.data_ptr(), kk.data_ptr(), v.data_ptr()) for q, kk, v in layers]

    def step(i):
        q, kk, v = ptrs[i % len(ptrs)]
        return lib.dcr_sparse_decode(q, kk, v, code, out.data_ptr(), None, B, H, Hkv, N, N, D, k,
                                     1e-12, ws.data_ptr(), ws_bytes, stream)

    path_codes = {"auto": _lib.PATH_AUTO, "classic": _lib.PATH_CLASSIC, "fused": _lib.PATH_FUSED,
                  "union": _lib.PATH_UNION}
    path_code = path_codes[args.sparse_path]
    _lib.set_sparse_path(path_code)
    _lib.set_score_form(_lib.SCORE_VALU if args.score_form == "valu" else _lib.SCORE_AUTO)
    variants = {"sparse": lambda i: _lib.check(step(i), "dcr_sparse_decode")}

    def on_path(other):
        # the same entry point held to another launch sequence for these steps
        def run(i):
            _lib.set_sparse_path(path_codes[other])
            try:
                _lib.check(step(i), "dcr_sparse_decode")
            finally:
                _lib.set_sparse_path(path_code)
        return run

    if not args.no_comparators:
        for other in ("fused", "union"):
            if other == args.sparse_path:
                continue
            if other == "fused":
                _lib.set_sparse_path(_lib.PATH_FUSED)
                one = lib.dcr_sparse_decode_launches(B, H, Hkv, N, D, k, code) == 1
                _lib.set_sparse_path(path_code)
                if not one:
                    continue
            variants[f"sparse_{other}"] = on_path(other)
    if not args.no_comparators:
        variants.update(comparator_steps(torch, _lib, lib, layers, cfg))

    for name, fn in variants.items():
        n_w = args.warmup if name.startswith("sparse") else min(args.warmup, 10)
        for i in range(n_w):
            fn(i)
    torch.cuda.synchronize()

    # ---- timed region: the reference's protocol (README.md:25-26), warm-up
    # then `sessions` sessions, each timing every variant over its steps in a
    # freshly shuffled order; `value` is the median over sessions of the
    # sparse path's mean per step (K steps per session, HIP events on the
    # launch stream, synchronised on both sides).
    rng = random.Random(args.seed)
    per_session = {name: [] for name in variants}
    t_wall = time.perf_counter()
    for sess in range(args.sessions):
        order = list(variants)
        rng.shuffle(order)
        for name in order:
            n = args.steps if name.startswith("sparse") or name == "dense_hip" else max(10, args.steps // 10)
            per_session[name].append(time_steps(torch, variants[name], n))
        print(f"[bench] session {sess + 1}/{args.sessions} ({' '.join(order)}): "
              f"sparse {per_session['sparse'][-1]:.2f} us", file=sys.stderr, flush=True)
    wall_s = time.perf_counter() - t_wall
    us_per_layer = statistics.median(per_session["sparse"])

    # ---- per-kernel durations (a further pass, events attached to each launch) ----
    with _lib.KernelTimer() as kt:
        for i in range(args.steps):
            step(i)
    per_kernel = {name: tot / n for name, (tot, n) in kt.result.items()}

    traffic = load_traffic(cfg.name)
    # Algorithmic bytes per launch, by the reference algorithm's accounting:
    #   score pass  K streamed once, B*Hkv*N*D*s (the 16-bit keys it writes are
    #               select overhead, below);
    #   select      overhead, not algorithmic: the keys read, B*H*N*2, and the
    #               indices written, B*H*k*4;
    #   attention   the reference gathers K and V rows per query head,
    #               B*H*k*D*s*2; this kernel gathers V rows and rebuilds the
    #               logits from each selected position's key and residual byte
    #               (fp16/bf16), B*H*k*(D*s + 3) -- both are reported.
    score_bytes = B * Hkv * N * D * esz
    select_bytes = B * H * N * 2 + B * H * k * 4
    ref_gather_bytes = B * H * k * D * esz * 2
    own_gather_bytes = ref_gather_bytes if dt == torch.float32 else B * H * k * (D * esz + 3)
    total_bytes = score_bytes + ref_gather_bytes
    stage_bytes = {"score_kernel": (score_bytes, "K once (B*Hkv*N*D*s)"),
                   "select_kernel": (select_bytes, "overhead: keys read (B*H*N*2) + indices written "
                                                   "(B*H*k*4)"),
                   "attn_kernel": (own_gather_bytes, "V rows + key and residual byte per selected "
                                                     "position (B*H*k*(D*s+3))" if dt != torch.float32
                                   else "K and V rows per selected position (B*H*k*D*s*2)"),
                   "union_attn_kernel": (ref_gather_bytes, "gather-attention as the reference algorithm "
                                                           "counts it: K and V rows per selected position "
                                                           "and query head (B*H*k*D*s*2); the kernel reads "
                                                           "the key and residual byte of every position "
                                                           "and head (B*H*N*3) and each V row its group "
                                                           "selected once"),
                   "fused_kernel": (total_bytes, "the whole step in one launch, select fused: K once "
                                                 "(B*Hkv*N*D*s) + K and V rows per selected position "
                                                 "and query head (B*H*k*D*s*2)")}
    stages = {}
    for name, us in per_kernel.items():
        st = {"us": round(us, 3)}
        if name in stage_bytes:
            nbytes, what = stage_bytes[name]
            gbps = nbytes / (us * 1e3)
            st.update(bytes=nbytes, bytes_definition=what, gbps=round(gbps, 1),
                      frac=round(gbps / HBM_PEAK_GBPS, 4))
        if name == "fused_kernel":
            st.update(own_bytes=score_bytes + own_gather_bytes,
                      own_bytes_definition="K once + V rows and key/residual per selected position "
                                           "and query head, before the kernel's per-group dedup")
        if name == "attn_kernel":
            st.update(reference_gather_bytes=ref_gather_bytes,
                      reference_gather_frac=round(ref_gather_bytes / (us * 1e3) / HBM_PEAK_GBPS, 4))
        if traffic.get(name) is not None:
            st["hbm_traffic_bytes"] = traffic[name]
            st["hbm_traffic_gbps"] = round(traffic[name] / (us * 1e3), 1)
        stages[name] = st
    dom = max(("score_kernel", "attn_kernel", "union_attn_kernel", "fused_kernel"),
              key=lambda n: per_kernel.get(n, 0.0))
    dom_bytes = stage_bytes[dom][0]
    achieved = dom_bytes / (per_kernel[dom] * 1e3)
    roofline = {"kernel": dom, "bound": "hbm", "achieved": round(achieved, 1),
                "peak": HBM_PEAK_GBPS, "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBPS, 4),
                "traffic": traffic.get(dom), "algorithmic_bytes": dom_bytes,
                "algorithmic_definition": stage_bytes[dom][1],
                "duration_us": round(per_kernel[dom], 3),
                "duration_source": "HIP events attached to each launch of the kernel "
                                   "(hipExtLaunchKernelGGL start/stop) on its launch stream"}
    if traffic.get(dom) is not None:
        roofline["traffic_source"] = f"profiles/hbm_traffic_{cfg.name}.txt (rocprofv3 --pmc)"
    path_gbps = total_bytes / (us_per_layer * 1e3)
    hbm = {"algorithmic_bytes": total_bytes,
           "definition": "reference algorithm: K once + gathered K and V rows per query head",
           "gbps": round(path_gbps, 1),
           "frac_of_peak": round(path_gbps / HBM_PEAK_GBPS, 4),
           "target_us_at_60pct": round(total_bytes / (0.6 * HBM_PEAK_GBPS * 1e3), 2)}
    if traffic and all(n in traffic for n in per_kernel):
        moved = sum(traffic[n] for n in per_kernel)
        hbm.update(measured_traffic_bytes=moved,
                   measured_traffic_gbps=round(moved / (us_per_layer * 1e3), 1),
                   measured_traffic_frac=round(moved / (us_per_layer * 1e3) / HBM_PEAK_GBPS, 4),
                   measured_traffic_source=f"profiles/hbm_traffic_{cfg.name}.txt (rocprofv3 --pmc, "
                                           "sum over the path's kernels)")

    result = {
        "metric": "sparse decode attn us/layer + HBM GB/s (% peak), N=32K B=4 c=0.15",
        "value": round(us_per_layer, 3),
        "unit": "us/layer",
        "n_gpus": 1, "steps": args.steps, "warmup": args.warmup, "sessions": args.sessions,
        "ms_per_step": round(us_per_layer / 1000.0, 5),
        "higher_is_better": False, "scaling": "weak", "vs_baseline": None,
        "dtype": "f32", "data": "synthetic",
        "config": {"workload": f"{cfg.name}: single-layer sparse decode op, Llama-3.2-1B heads "
                               f"(32 Q / 8 KV, D=64), B={B}, N={N}, c={cfg.c}, k={k}, "
                               f"{str(dt).replace('torch.', '')} K/V, fp32 accumulation",
                   "B": B, "N": N, "H": H, "Hkv": Hkv, "D": D, "k": k,
                   "kv_dtype": str(dt).replace("torch.", ""), "layers_rotated": args.layers,
                   "parallelism": "single GPU"},
        "timing": {"protocol": f"{args.warmup} warm-up steps, then {args.sessions} sessions, each "
                               "timing every variant in a shuffled order (the reference's 50 warm-up "
                               "/ 30 timed / 3 randomized-order sessions, README.md:25-26); value = "
                               "median of the sessions' sparse means",
                   "sparse_us_per_session": [round(x, 3) for x in per_session["sparse"]],
                   "timed_wall_s": round(wall_s, 3)},
        "score_form": args.score_form,
        "sparse_path": {"setting": args.sparse_path,
                        "launches": lib.dcr_sparse_decode_launches(B, H, Hkv, N, D, k, code)},
        "hbm": hbm,
        "stages": stages,
        "roofline": roofline,
    }

    if not args.no_comparators:
        result["comparators"] = comparator_summary(torch, per_session, cfg)
    if args.configs:
        result["other_configs"] = other_configs(torch, _lib, lib)
        result["rank_local"] = rank_local_bench(torch)
    del layers, variants
    torch.cuda.empty_cache()
    if not args.no_e2e:
        result["e2e"] = e2e_decode(torch, args.e2e_steps)
    if not args.no_cpu_baseline:
        base = cpu_baselines(torch, cfg, args.cpu_seconds)
        result["cpu_baseline"] = base["torch_reference_calls"]
        result["cpu_baseline_c_port"] = base["c_oracle"]
    result["env"] = env_stamp(torch)
    print(json.dumps(result), flush=True)


def time_steps(torch, fn, n):
    """Mean us per call of fn(i) over n calls: synchronise, HIP events around
    the calls on the current stream, synchronise."""
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for i in range(n):
        fn(i)
    e1.record()
    torch.cuda.synchronize()
    return 1000.0 * e0.elapsed_time(e1) / n


def comparator_steps(torch, _lib, lib, layers, cfg):
    """Dense decode attention on the same GPU over the same layers: this
    build's dense HIP kernel, torch's fused SDPA and the reference's eager
    dense branch."""
    B, H, Hkv, N, D = cfg.B, cfg.H, cfg.Hkv, cfg.N, cfg.D
    dev = torch.device("cuda:0")
    code = _lib.DTYPE_CODE[cfg.dtype]
    stream = torch.cuda.current_stream().cuda_stream
    ws_bytes = lib.dcr_dense_decode_workspace_bytes(B, H, Hkv, N, D)
    ws = _lib.workspace(ws_bytes, dev)
    out = torch.empty(B, H, D, dtype=cfg.dtype, device=dev)

    def dense_hip(i):
        q, kk, v = layers[i % len(layers)]
        _lib.check(lib.dcr_dense_decode(q.data_ptr(), kk.data_ptr(), v.data_ptr(), code,
                                        out.data_ptr(), B, H, Hkv, N, N, D, ws.data_ptr(), ws_bytes,
                                        stream), "dcr_dense_decode")

    from dcr_attention_amd.llama.model import eager_sdpa

    def torch_eager(i):
        # The reference's dense branch as its latency tables ran it
        # (_sdpa_forward on repeat_kv-expanded K/V, fp32 softmax).
        q, kk, v = layers[i % len(layers)]
        eager_sdpa(q.unsqueeze(2), kk, v, H // Hkv)

    import torch.nn.functional as F

    def torch_sdpa(i):
        # torch's fused scaled_dot_product_attention on the un-repeated cache
        # (GQA), default backend selection.
        q, kk, v = layers[i % len(layers)]
        F.scaled_dot_product_attention(q.unsqueeze(2), kk, v, enable_gqa=True)

    return {"dense_hip": dense_hip, "torch_sdpa": torch_sdpa, "torch_eager": torch_eager}


def comparator_summary(torch, per_session, cfg):
    esz = torch.tensor([], dtype=cfg.dtype).element_size()
    dense_bytes = 2 * cfg.B * cfg.Hkv * cfg.N * cfg.D * esz
    res = {"dense_hip_us": round(statistics.median(per_session["dense_hip"]), 3),
           "dense_bytes": dense_bytes,
           "dense_bytes_definition": "K and V once (2*B*Hkv*N*D*s)"}
    res["dense_hip_gbps"] = round(dense_bytes / (res["dense_hip_us"] * 1e3), 1)
    res["dense_hip_frac"] = round(res["dense_hip_gbps"] / HBM_PEAK_GBPS, 4)
    res["torch_eager_sdpa_us"] = round(statistics.median(per_session["torch_eager"]), 3)
    res["torch_sdpa_us"] = round(statistics.median(per_session["torch_sdpa"]), 3)
    res["sparse_vs_dense_hip"] = round(res["dense_hip_us"] / statistics.median(per_session["sparse"]), 4)
    for name in per_session:
        if name.startswith("sparse_"):
            res[f"{name}_us"] = round(statistics.median(per_session[name]), 3)
    res["per_session_us"] = {n: [round(x, 3) for x in v] for n, v in per_session.items() if n != "sparse"}
    return res


def rank_local_bench(torch, cpu=True):
    """Rank-local window attention (kernel.hip.rank_local_fwd) at a decode
    shape (C2 heads, window = C2's k) and a prefill shape, against the
    reference's CPU path (rank_local_fwd_torch restated in oracle/torch_twin)
    on a bounded sample."""
    from dcr_attention_amd.kernel.hip.rank_local_fwd import rank_local_fwd_hip
    from oracle import torch_twin
    out = {}
    shapes = {"decode": (4, 32, 1, 32768, 64, 4916), "prefill": (1, 32, 4096, 4096, 64, 256)}
    for name, (B, H, Nq, Nkv, D, k) in shapes.items():
        g = torch.Generator(device="cuda").manual_seed(0)
        Q = torch.randn(B, H, Nq, D, device="cuda", generator=g).half()
        K = torch.randn(B, H, Nkv, D, device="cuda", generator=g).half()
        V = torch.randn(B, H, Nkv, D, device="cuda", generator=g).half()
        if Nq == Nkv:
            rc = torch.arange(Nq, device="cuda", dtype=torch.int32).expand(B, H, Nq).contiguous()
        else:
            rc = torch.randint(0, Nkv, (B, H, Nq), device="cuda", generator=g, dtype=torch.int32)
        for _ in range(5):
            rank_local_fwd_hip(Q, K, V, None, rc, k)
        torch.cuda.synchronize()
        n = 50
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(n):
            rank_local_fwd_hip(Q, K, V, None, rc, k)
        e1.record()
        torch.cuda.synchronize()
        us = 1000.0 * e0.elapsed_time(e1) / n
        rows = B * H * Nq * min(k + 1, Nkv)          # (query, key) pairs in the windows
        res = {"B": B, "H": H, "Nq": Nq, "Nkv": Nkv, "D": D, "k_window": k, "dtype": "float16",
               "hip_us": round(us, 2), "gflops": round(4.0 * rows * D / (us * 1e3), 1)}
        if Nq == 1:   # decode: each head streams its window of K and V rows once
            nbytes = B * H * min(k + 1, Nkv) * D * 2 * 2
            res["bytes"] = nbytes
            res["gbps"] = round(nbytes / (us * 1e3), 1)
        if not cpu:
            out[name] = res
            continue
        # the reference's CPU path on one (b, h) head (bounded sample), scaled
        qc, kc, vc, rcc = (Q[:1, :1].cpu(), K[:1, :1].cpu(), V[:1, :1].cpu(), rc[:1, :1].cpu())
        t0 = time.perf_counter()
        reps = 0
        while time.perf_counter() - t0 < 3.0 and reps < 20:
            torch_twin.rank_local_fwd(qc, kc, vc, rcc, k)
            reps += 1
        cpu_us = 1e6 * (time.perf_counter() - t0) / reps * B * H
        res["cpu_baseline"] = {"value": round(cpu_us, 1), "unit": "us", "cores": torch.get_num_threads(),
                               "kind": "port", "sample": f"one of {B * H} heads x {reps} reps, scaled x{B * H}; "
                               "rank_local_fwd_torch restated (oracle/torch_twin.py)"}
        out[name] = res
        del Q, K, V, rc
        torch.cuda.empty_cache()
    out["decode_api"] = rank_local_api_bench(torch)
    return out


def rank_local_api_bench(torch):
    """The public rank_local_attention at a decode step (C2 heads, window =
    C2's k, axis = each query's direction, un-repeated fp16 cache): sort
    bookkeeping + the kernel reading K/V through the sort permutation, against
    the reference's sequence (sorted copies of K and V, then the kernel)."""
    from dcr_attention_amd.kernel import sort_helpers as sh
    from dcr_attention_amd.kernel.hip.rank_local_fwd import rank_local_fwd_hip
    from dcr_attention_amd.kernel.rank_local_attention import _normalize_axis, rank_local_attention
    B, H, Hkv, N, D, k = 4, 32, 8, 32768, 64, 4916
    g = torch.Generator(device="cuda").manual_seed(0)
    Q = torch.randn(B, H, 1, D, device="cuda", generator=g).half()
    K = torch.randn(B, Hkv, N, D, device="cuda", generator=g).half()
    V = torch.randn(B, Hkv, N, D, device="cuda", generator=g).half()
    axis = Q.squeeze(2).float()

    def copies():
        idx = sh.prepare_sort_indices(Q, K, _normalize_axis(axis))
        Qs = sh.gather_by_sort_idx(Q, idx.sort_idx_q)
        o, _ = rank_local_fwd_hip(Qs, sh.gather_by_sort_idx(K, idx.sort_idx_k),
                                  sh.gather_by_sort_idx(V, idx.sort_idx_k), None, idx.r_center, k)
        return sh.scatter_by_inv_perm(o, idx.inv_q_perm)

    def inplace():
        return rank_local_attention(Q, K, V, axis, k_window=k)

    res = {"B": B, "H": H, "Hkv": Hkv, "Nkv": N, "D": D, "k_window": k, "dtype": "float16"}
    assert torch.equal(copies(), inplace())
    for name, fn in (("us_in_place", inplace), ("us_sorted_copies", copies)):
        for _ in range(3):
            fn()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(10):
            fn()
        e1.record()
        torch.cuda.synchronize()
        res[name] = round(1000.0 * e0.elapsed_time(e1) / 10, 1)
    del Q, K, V
    torch.cuda.empty_cache()
    return res


def other_configs(torch, _lib, lib):
    """The single-GPU op at the other benchmark configurations (C1, C4a-c, C5,
    each at its own batch size): sparse path vs the dense HIP kernel, us/layer."""
    from dcr_attention_amd.synthetic import CONFIGS, make_qkv
    out = {}
    stream = torch.cuda.current_stream().cuda_stream
    for name in ("C1", "C4a", "C4b", "C4c", "C5"):
        cfg = CONFIGS[name]
        B = cfg.B
        H, Hkv, N, D, k, dt = cfg.H, cfg.Hkv, cfg.N, cfg.D, cfg.k, cfg.dtype
        code = _lib.DTYPE_CODE[dt]
        nl = 3
        lay = [make_qkv(B, H, Hkv, N, D, dt, seed=l, device="cuda", n_sinks=cfg.n_sinks,
                        n_outlier=cfg.n_outlier) for l in range(nl)]
        o = torch.empty(B, H, D, dtype=dt, device="cuda")
        nws = lib.dcr_sparse_decode_workspace_bytes(B, H, Hkv, N, D, k, code)
        ws = _lib.workspace(nws, torch.device("cuda:0"))
        ndw = lib.dcr_dense_decode_workspace_bytes(B, H, Hkv, N, D)
        dws = _lib.workspace(ndw, torch.device("cuda:0"))

        def sp(i):
            q, kk, v = lay[i % nl]
            _lib.check(lib.dcr_sparse_decode(q.data_ptr(), kk.data_ptr(), v.data_ptr(), code,
                                             o.data_ptr(), None, B, H, Hkv, N, N, D, k, 1e-12,
                                             ws.data_ptr(), nws, stream), "dcr_sparse_decode")

        def dn(i):
            q, kk, v = lay[i % nl]
            _lib.check(lib.dcr_dense_decode(q.data_ptr(), kk.data_ptr(), v.data_ptr(), code,
                                            o.data_ptr(), B, H, Hkv, N, N, D, dws.data_ptr(), ndw,
                                            stream), "dcr_dense_decode")

        def t(fn, n=30):
            for i in range(5):
                fn(i)
            torch.cuda.synchronize()
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
            for i in range(n):
                fn(i)
            e1.record()
            torch.cuda.synchronize()
            return round(1000.0 * e0.elapsed_time(e1) / n, 2)

        out[name] = {"B": B, "N": N, "k": k, "dtype": str(dt).replace("torch.", ""),
                     "launches": lib.dcr_sparse_decode_launches(B, H, Hkv, N, D, k, code),
                     "sparse_us": t(sp), "dense_hip_us": t(dn)}
        prev = _lib.set_sparse_path(_lib.PATH_CLASSIC)
        try:
            out[name]["sparse_classic_us"] = t(sp)
            _lib.set_sparse_path(_lib.PATH_UNION)
            out[name]["sparse_union_us"] = t(sp)
            _lib.set_sparse_path(_lib.PATH_FUSED)
            if lib.dcr_sparse_decode_launches(B, H, Hkv, N, D, k, code) == 1:
                out[name]["sparse_fused_us"] = t(sp)
        finally:
            _lib.set_sparse_path(prev)
        del lay, ws, dws
        torch.cuda.empty_cache()
    return out


def e2e_decode(torch, steps):
    """C3: Llama-3.2-1B-shaped decoder (16 layers, random fp16 weights), B=4,
    KV cache of 32768 synthetic positions, greedy decode steps.  Attention
    per layer: the DCR branch (this path, k_eff = adaptive_k_window), the dense
    HIP decode kernel, or the reference's eager dense branch (repeat_kv +
    matmul + fp32 softmax).  Everything else in the step is identical."""
    from dcr_attention_amd.llama import DCRLlamaConfig
    from dcr_attention_amd.llama.model import LLAMA_3_2_1B, DCRLlamaDecoder, KVCache
    B, n_ctx = 4, 32768
    cfg = LLAMA_3_2_1B
    dec = DCRLlamaDecoder(cfg, dtype=torch.float16, device="cuda").init_random(0)
    cache = KVCache.allocate(cfg, B, n_ctx + 4 * (steps + 8), torch.float16, "cuda")
    cache.fill_synthetic(n_ctx, seed=1)
    modes = {"dcr": (DCRLlamaConfig(), False), "dense_hip": (DCRLlamaConfig(enable_dcr=False), False),
             "torch_eager": (DCRLlamaConfig(enable_dcr=False), True)}
    out = {"config": f"C3: Llama-3.2-1B shapes, {cfg.num_layers} layers, B={B}, cache {n_ctx} "
                     f"positions (synthetic), fp16, greedy decode", "steps": steps}
    def timed(fn, n):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(n):
            fn()
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / n

    for name, (dcfg, eager) in modes.items():
        dec.dcr, dec.eager_attention = dcfg, eager
        cache.length = n_ctx
        tok = torch.ones(B, dtype=torch.long, device="cuda")
        for _ in range(3):
            tok = dec.decode_step(tok, cache)
        torch.cuda.synchronize()
        DCRLlamaDecoder.reset_counters()
        state = {"tok": tok}

        def eager_step():
            state["tok"] = dec.decode_step(state["tok"], cache)
        out[f"{name}_ms_per_step"] = round(timed(eager_step, steps), 4)
        out[f"{name}_branch_counts"] = DCRLlamaDecoder.get_counters()

        # The same step captured in a HIP graph (launch overhead removed): one
        # decode step at a fixed position, replayed; the logits of every
        # replay are checked against the eager step at that position.
        pos = cache.length
        tok_in = state["tok"].view(-1, 1).clone()
        ref = dec.forward(tok_in, cache)
        cache.length = pos
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):  # warm up on the capture stream
            dec.forward(tok_in, cache)
            cache.length = pos
        torch.cuda.current_stream().wait_stream(side)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            logits = dec.forward(tok_in, cache)
        cache.length = pos
        ok = True
        for _ in range(3):
            graph.replay()
            torch.cuda.synchronize()
            ok = ok and bool(torch.allclose(logits, ref, atol=1e-2, rtol=0))
        out[f"{name}_graph_ms_per_step"] = round(timed(graph.replay, steps), 4)
        out[f"{name}_graph_replays_match_eager"] = ok
        del graph, logits, ref
    for suffix in ("", "_graph"):
        d = out[f"dcr{suffix}_ms_per_step"]
        out[f"speedup{suffix}_vs_dense_hip"] = round(out[f"dense_hip{suffix}_ms_per_step"] / d, 3)
        out[f"speedup{suffix}_vs_torch_eager"] = round(out[f"torch_eager{suffix}_ms_per_step"] / d, 3)
    return out


def cpu_baselines(torch, cfg, seconds):
    """The reference's CPU path on the host, on a bounded sample of the workload.

    torch_reference_calls: the reference's M1 path
      (topk_qaxis_attention_reference, qaxis_topk_reference.py:200-259) restated
      with the same torch calls (oracle/torch_twin.sparse_decode: linalg.norm,
      einsum, stable argsort, gather, 64-row online softmax), torch's CPU
      thread pool;
    c_oracle: the C restatement (oracle/dcr_oracle.c, OpenMP).
    Sample: the same configuration with B=1 (one quarter of a C2 layer), repeated
    for about `seconds` each, scaled to one full layer (x B)."""
    from oracle import cpu, torch_twin
    from dcr_attention_amd.synthetic import make_inputs
    Q, K, V = make_inputs(cfg, seed=0, B=1)
    out = {}
    omp = int(os.environ.get("OMP_NUM_THREADS", "0")) or len(os.sched_getaffinity(0))
    for name, fn, cores, what in (
            ("torch_reference_calls", lambda: torch_twin.sparse_decode(Q, K, V, cfg.k),
             torch.get_num_threads(), "the reference's M1 torch calls (oracle/torch_twin.py)"),
            ("c_oracle", lambda: cpu.sparse_decode(Q, K, V, cfg.k), omp,
             "C restatement of M1 (oracle/dcr_oracle.c, OpenMP)")):
        fn()  # warm (page in, thread pools)
        reps, t0 = 0, time.perf_counter()
        while True:
            fn()
            reps += 1
            el = time.perf_counter() - t0
            if el >= seconds or reps >= 5000:
                break
        us_sample = 1e6 * el / reps
        out[name] = {"value": round(us_sample * cfg.B, 1), "unit": "us/layer", "cores": cores,
                     "kind": "port",
                     "sample": f"{cfg.name} with B=1 (1/{cfg.B} of a layer), {reps} reps in {el:.1f} s, "
                               f"scaled x{cfg.B}; {what}"}
    return out


if __name__ == "__main__":
    main()
