"""Benchmark of the SignRot W4A4 QLinear hot path on one MI355X.

Default workload (config 2, the one the headline metric is quoted on):
Llama-3-8B down_proj W4A4 prefill, M=2048 tokens, K=14336, N=4096.
One step = one QLinear forward over one batch:
  had_sign_quant  (had_28 ⊗ H_512 rotation, SignRot sign, per-token int4
                   quantization + packing: one launch)
  w4a4_linear     (int4 x int4 GEMM on the int8 MFMA + per-token x
                   per-channel fp16 dequant epilogue: one launch)
Inputs are resident in HBM before the timed region; the step rotates over
several distinct input/weight sets (> 512 MB in total) so no step is served
from the 256 MB MALL.

Prints ONE JSON line (rank 0).  --gpus N > 1 exits: this build runs on one
GPU.  The CPU baseline is the reference's PyTorch fake-quant simulation of
the same path (restated in oracle/fakequant.py), timed on the host cores on
a bounded row sample.
"""
import argparse
import json
import math
import os
import sys
import time

import torch

METRIC = "W4A4 QLinear TOPS (M=2048) + decode µs/layer; % of MI355X roofline"
PEAK_INT8_TOPS = 5000.0   # MI355X dense int8 MFMA, 5.0 POPS
PEAK_HBM_GBS = 8000.0     # MI355X HBM3E, 8 TB/s
PEAK_FP6_TOPS = 10100.0   # MI355X dense fp6 / fp4 MFMA, 10.1 PFLOPS (the bf6 path's MFMA)


def parse():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=50)
    p.add_argument("--warmup", type=int, default=10)
    p.add_argument("--M", type=int, default=2048)
    p.add_argument("--K", type=int, default=14336)
    p.add_argument("--N", type=int, default=4096)
    p.add_argument("--outliers", type=int, default=8)
    p.add_argument("--outlier-mag", type=float, default=50.0)
    p.add_argument("--seed", type=int, default=1)
    p.add_argument("--no-cpu-baseline", action="store_true")
    p.add_argument("--no-decode", action="store_true",
                   help="skip the config-3 decode-layer measurement")
    p.add_argument("--decode-layers", type=int, default=4,
                   help="distinct layers (weights + cache) replayed per decode step")
    p.add_argument("--decode-steps", type=int, default=20)
    p.add_argument("--no-configs", action="store_true",
                   help="skip the per-config measurements (cfg1, cfg2 sweep, cfg4, cfg5)")
    p.add_argument("--calibrate-copy", action="store_true",
                   help="only run plain device copies of a known size (the reference "
                        "kernel for scaling the FETCH_SIZE / WRITE_SIZE counters)")
    p.add_argument("--prefill-attention-only", action="store_true",
                   help="only measure the prefill attention (Llama-70B heads, T = 512, "
                        "2048, 8192) and print its results")
    p.add_argument("--profile", choices=PROFILE_WORKLOADS, default=None,
                   help="only run one workload a few times (for rocprofv3 counter passes): "
                        "the cfg2 QLinear at M = 2048, 128, 16 or 8192, the cfg4 MLP at M = "
                        "512, the cfg5 MoE block, the cfg3 decode layer, the prefill attention "
                        "(Llama-70B heads, T = 8192) or the cfg2 QLinear on the bf6 path at "
                        "M = 2048")
    p.add_argument("--cpu-rows", type=int, default=256,
                   help="rows of the CPU baseline sample")
    p.add_argument("--min-bytes", type=float, default=640e6,
                   help="distinct input bytes to rotate over (defeats the MALL)")
    return p.parse_args()


def make_inputs(args, dev):
    """Synthetic cfg2 tensors: X N(0,1) fp16 with seeded outlier channels;
    sign from the calibration rule on the rotated X; W N(0, 0.02) fp16 with
    the sign folded by column, RTN per-channel symmetric int4."""
    from signrot_amd import _CUDA
    from signrot_amd.functional.hadamard import adj_sign_from_rotated, get_hadK
    from signrot_amd.functional.quantization import rtn_weight_pack

    M, K, N = args.M, args.K, args.N
    g = torch.Generator().manual_seed(args.seed)
    x = torch.randn(M, K, generator=g)
    ch = torch.randperm(K, generator=g)[: args.outliers]
    sg = torch.randint(0, 2, (args.outliers,), generator=g).float() * 2 - 1
    x[:, ch] *= sg * args.outlier_mag
    x = x.half().to(dev)
    had, k = get_hadK(K)
    hadk = had.half().to(dev).contiguous() if k > 1 else None
    # sign-adjust vector (fake_quant/quant_utils.py:362-367) on the rotated X
    sign = adj_sign_from_rotated(_CUDA.online_hadamard(x, hadk, k, None)).contiguous()
    # weights: N(0, 0.02), fold sign, RTN on the symmetric grid (A18 rule)
    w = (torch.randn(N, K, generator=g) * 0.02).half().to(dev)
    wq, s16, wfq = rtn_weight_pack(w * sign, symmetric_grid=True)
    return x, hadk, k, sign, wq, s16, wfq


def time_cpu_baseline(args, x, hadk, k, sign, wfq):
    """Reference fake-quant path on the host cores over a row sample."""
    sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))
    from oracle import fakequant
    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    rows = min(args.cpu_rows, args.M)
    xc = x[:rows].cpu()
    hc = hadk.float().cpu() if hadk is not None else None
    sc = sign.cpu()
    wc = wfq.cpu()
    fakequant.qlinear(xc[:8], hc, k, sc, wc)  # warmup
    reps, times = 0, []
    t_end = time.perf_counter() + 20.0
    while reps < 10 and (reps < 3 or time.perf_counter() < t_end):
        t0 = time.perf_counter()
        fakequant.qlinear(xc, hc, k, sc, wc)
        times.append(time.perf_counter() - t0)
        reps += 1
    t = sum(times) / len(times)
    sd = (sum((v - t) ** 2 for v in times) / max(1, len(times) - 1)) ** 0.5
    tops = 2.0 * rows * args.N * args.K / t / 1e12
    return {"value": tops, "unit": "TOPS", "cores": cores, "cpu_model": cpu_model(),
            "kind": "port",
            "sample": (f"{rows} of {args.M} rows of the same QLinear (fp16 fake-quant: "
                       f"matmul_hadU + sign + per-token sym int4 quant-dequant + F.linear), "
                       f"{reps} reps, {t * 1e3:.1f} ms +- {1.96 * sd * 1e3:.1f} ms each")}


COPY_BYTES = 1 << 30
PROFILE_WORKLOADS = ("cfg2_M2048", "cfg2_M128", "cfg2_M8192", "cfg2_M16", "cfg4_M512",
                     "cfg5_moe", "cfg3_decode", "prefill_T8192", "cfg2_bf6_M2048")


def bench_decode_layer(args, dev):
    """Config 3: one Llama-3-8B-shape decoder layer in real-quant decode
    (hidden 4096, 32 query / 8 KV heads of 128, FFN 14336, batch 32, 4096
    cached tokens, one new token per sequence).  `decode_layers` distinct
    layers (own weights, own cache layer) run back to back inside one HIP
    graph, so weights and KV pages stream from HBM as in a full model;
    returns microseconds per layer and the per-layer HBM floor."""
    from signrot_amd.transformers import MultiLayerPagedKVCache4Bit
    from signrot_amd.transformers.decode_layer import W4A4LlamaDecodeLayer, rope_cos_sin
    B, T, hidden, Hq, Hkv, D, ffn, page = 32, 4096, 4096, 32, 8, 128, 14336, 256
    NL = args.decode_layers
    layers = [W4A4LlamaDecodeLayer.random(hidden, Hq, Hkv, D, ffn, layer_idx=i, seed=args.seed + i,
                                          device=dev) for i in range(NL)]
    cache = MultiLayerPagedKVCache4Bit(B, page, T + page, dev, NL, Hkv, D, group_size=Hq // Hkv)
    # seeded random int4 context: codes and [scale, zero] pairs of T tokens
    gen = torch.Generator(device=dev).manual_seed(args.seed)
    cache.pages.copy_(torch.randint(0, 256, cache.pages.shape, dtype=torch.uint8, device=dev,
                                    generator=gen))
    cache.scales[..., 0].uniform_(0.02, 0.3, generator=gen)
    cache.scales[..., 1].uniform_(-2.0, 2.0, generator=gen)
    cache.mark_prefilled(T)
    h0 = (torch.randn(B, 1, hidden, device=dev, generator=gen) * 0.5).half()
    cos, sin = rope_cos_sin([T], D, layers[0].rope_theta, dev)
    # the reference's graph protocol (kv_cache.py:435-460): index buffers are
    # refreshed outside the graph and frozen inside it
    cache.refresh_specs(T + 1)
    cache.freeze_specs(True)

    def step():
        cache.length = T
        h = h0
        for layer in layers:
            h = layer(h, cache, cos, sin)
        return h

    eager = step()
    for _ in range(2):
        step()
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        step()
    torch.cuda.current_stream().wait_stream(side)
    with torch.cuda.graph(graph):
        out = step()
    for _ in range(3):
        graph.replay()
    torch.cuda.synchronize()
    assert torch.equal(out, eager), "graph replay differs from the eager decode step"
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(args.decode_steps):
        graph.replay()
    e1.record()
    torch.cuda.synchronize()
    us_layer = e0.elapsed_time(e1) * 1e3 / args.decode_steps / NL
    wbytes = sum(getattr(layers[0], f"w_{n}").numel() for n in ("qkv", "o", "gu", "down"))
    kvbytes = B * T * Hkv * 2 * (D // 2 + 4)
    hbm = wbytes + kvbytes
    return {
        "workload": ("cfg3 Llama-3-8B-shape W4A4 decoder layer, decode step: batch 32, "
                     "4096-token int4 KV context (GQA 32/8), FFN 14336, HIP graph"),
        "us_per_layer": round(us_layer, 2),
        "layers_per_step": NL,
        "hbm_bytes_per_layer": hbm,
        "achieved_GBs": round(hbm / (us_layer * 1e-6) / 1e9, 1),
        "frac_hbm": round(hbm / (us_layer * 1e-6) / 1e9 / PEAK_HBM_GBS, 4),
        "floor_us_at_peak": round(hbm / (PEAK_HBM_GBS * 1e9) * 1e6, 2),
    }


def _time_launches(launch, n, stream):
    """Average ms of `launch(i)`, i = 0 .. n-1, back to back, HIP events on
    the launch stream."""
    for i in range(2):
        launch(i)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    for i in range(n):
        launch(i)
    e1.record(stream)
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / n


def _time_graph(launch, n, reps=5):
    """Ms per launch of `launch(i)`, i = 0 .. n-1, captured once into a HIP
    graph: the median over `reps` replays, each between its own HIP events
    (one disturbed replay, e.g. a clock-state change, does not move it) --
    the launches' GPU time without the host's per-call cost, which is of
    the order of the small-M kernels themselves.  `launch` must issue its
    work on the current stream."""
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for i in range(2):
            launch(i)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for i in range(n):
            launch(i)
    graph.replay()
    torch.cuda.synchronize()
    st = torch.cuda.current_stream()
    ev = [torch.cuda.Event(enable_timing=True) for _ in range(reps + 1)]
    ev[0].record(st)
    for r in range(reps):
        graph.replay()
        ev[r + 1].record(st)
    torch.cuda.synchronize()
    del graph
    per = sorted(ev[r].elapsed_time(ev[r + 1]) for r in range(reps))
    return per[reps // 2] / n


def _roof(us, ops, nbytes):
    tops = ops / (us * 1e-6) / 1e12
    gbs = nbytes / (us * 1e-6) / 1e9
    bound = "mfma" if ops / (PEAK_INT8_TOPS * 1e12) > nbytes / (PEAK_HBM_GBS * 1e9) else "hbm"
    return {"us": round(us, 2), "TOPS": round(tops, 1), "GBs": round(gbs, 1),
            "frac_mfma": round(tops / PEAK_INT8_TOPS, 4), "frac_hbm": round(gbs / PEAK_HBM_GBS, 4),
            "bound": bound, "algorithmic_ops": ops, "algorithmic_bytes": nbytes}


def _rand_w(n, k, dev, g):
    return torch.randint(0, 256, (n, k // 2), dtype=torch.uint8, device=dev, generator=g)


def bench_qlinear(dev, M, K, N, seed, n_out=8, mag=50.0, min_bytes=2.2e9, reps=20):
    """One W4A4 QLinear (had_sign_quant + w4a4_linear) at [M, K] x [N, K]:
    whole-QLinear and per-kernel averages over distinct input/weight sets
    (> min_bytes in total, so weights stream from HBM, not the MALL), timed
    as launches replayed from a HIP graph (the serving loop's form; the
    eager back-to-back time of the whole QLinear is reported beside it)."""
    from signrot_amd import _native
    from signrot_amd.functional.hadamard import get_hadK
    st = torch.cuda.current_stream()
    g = torch.Generator(device=dev).manual_seed(seed)
    had, k = get_hadK(K)
    hadk = had.half().to(dev).contiguous() if k > 1 else None
    sign = (torch.randint(0, 2, (K,), device=dev, generator=g).to(torch.int8) * 2 - 1)
    set_bytes = M * K * 2 + N * K // 2 + M * K // 2 + M * N * 2
    nsets = max(1, min(256, math.ceil(min_bytes / set_bytes)))
    x0 = torch.randn(M, K, device=dev, generator=g)
    ch = torch.randperm(K, device=dev, generator=g)[:n_out]
    x0[:, ch] *= mag
    x0 = x0.half()
    xs = [x0] + [x0.clone() for _ in range(min(nsets, 8) - 1)]
    ws = [_rand_w(N, K, dev, g) for _ in range(nsets)]
    wsc = (torch.rand(N, device=dev, generator=g) * 1e-3 + 1e-4).half()
    qb = [torch.empty(M, K // 2, dtype=torch.uint8, device=dev) for _ in range(len(xs))]
    sb = [torch.empty(M, dtype=torch.float16, device=dev) for _ in range(len(xs))]
    ob = [torch.empty(M, N, dtype=torch.float16, device=dev) for _ in range(len(xs))]
    hp = hadk.data_ptr() if hadk is not None else None
    # the split-K workspace the library asks for at this shape (0: none),
    # allocated once, outside the timed loops
    ws_bytes = int(_native.lib().srq_w4a4_linear_ws_bytes(M, N, K))
    wsp = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=dev)

    def had(i):
        j = i % len(xs)
        _native.call("srq_had_sign_quant", xs[j].data_ptr(), M, K, k, hp, sign.data_ptr(), 0,
                     1.0, qb[j].data_ptr(), sb[j].data_ptr(),
                     torch.cuda.current_stream().cuda_stream)

    def gemm(i):
        j = i % len(xs)
        _native.call("srq_w4a4_linear_ws", qb[j].data_ptr(), sb[j].data_ptr(),
                     ws[i % nsets].data_ptr(), wsc.data_ptr(), None, M, N, K, ob[j].data_ptr(),
                     wsp.data_ptr(), ws_bytes, torch.cuda.current_stream().cuda_stream)

    def both(i):
        had(i)
        gemm(i)

    n = max(reps, min(nsets, 64))
    t_eager = _time_launches(both, n, st) * 1e3
    t_all = _time_graph(both, n) * 1e3
    t_had = _time_graph(had, n) * 1e3
    t_gemm = _time_graph(gemm, n) * 1e3
    ops = 2.0 * M * N * K
    res = {"M": M, "K": K, "N": N, "hadamard": f"had_{k} x H_{K // k}", "weight_sets": nsets,
           "timing": "hip_graph", "qlinear_eager_us": round(t_eager, 2),
           "qlinear": _roof(t_all, ops, M * K * 2 + N * K // 2 + M * N * 2 + M * 2 + N * 2),
           "had_sign_quant": _roof(t_had, 0.0, M * K * 2 + M * K // 2 + M * 2),
           "w4a4_linear": _roof(t_gemm, ops, M * K // 2 + N * K // 2 + M * N * 2 + M * 2 + N * 2)}
    res["gemm_kernel"] = gemm_kernel_name(M, N, K, ws_bytes > 0)
    del xs, ws, qb, sb, ob, wsp
    torch.cuda.empty_cache()
    return res


def bench_qlinear_asym(dev, M, K, N, seed, n_out=8, mag=50.0, min_bytes=2.2e9):
    """The cfg2 QLinear with asymmetric activations (the signrot preset's
    --a_asym): had_sign_asym_quant (rotation + sign + uint4 quantizer with
    per-token zero points) + w4a4_linear_asym (unsigned-A GEMM, zero
    correction, dequant), per-kernel and whole-QLinear averages."""
    from signrot_amd import _native
    from signrot_amd.functional.hadamard import get_hadK
    st = torch.cuda.current_stream()
    g = torch.Generator(device=dev).manual_seed(seed)
    had, k = get_hadK(K)
    hadk = had.half().to(dev).contiguous()
    sign = (torch.randint(0, 2, (K,), device=dev, generator=g).to(torch.int8) * 2 - 1)
    set_bytes = M * K * 2 + N * K // 2 + M * K // 2 + M * N * 2
    nsets = max(1, min(256, math.ceil(min_bytes / set_bytes)))
    x0 = torch.randn(M, K, device=dev, generator=g)
    ch = torch.randperm(K, device=dev, generator=g)[:n_out]
    x0[:, ch] *= mag
    x0 = (x0 + 0.5).half()
    xs = [x0] + [x0.clone() for _ in range(min(nsets, 8) - 1)]
    wts = [_rand_w(N, K, dev, g) for _ in range(nsets)]
    wsum = [torch.empty(N, dtype=torch.int32, device=dev) for _ in range(nsets)]
    for w, ws in zip(wts, wsum):
        _native.call("srq_sum_i4", w.data_ptr(), N, K // 2, 1, ws.data_ptr(), st.cuda_stream)
    wsc = (torch.rand(N, device=dev, generator=g) * 1e-3 + 1e-4).half()
    qb = [torch.empty(M, K // 2, dtype=torch.uint8, device=dev) for _ in range(len(xs))]
    sb = [torch.empty(M, dtype=torch.float16, device=dev) for _ in range(len(xs))]
    zb = [torch.empty(M, dtype=torch.float16, device=dev) for _ in range(len(xs))]
    zi = [torch.empty(M, dtype=torch.int8, device=dev) for _ in range(len(xs))]
    ob = [torch.empty(M, N, dtype=torch.float16, device=dev) for _ in range(len(xs))]

    def had(i):
        j = i % len(xs)
        _native.call("srq_had_sign_asym_quant", xs[j].data_ptr(), M, K, k, hadk.data_ptr(),
                     sign.data_ptr(), 1.0, qb[j].data_ptr(), sb[j].data_ptr(), zb[j].data_ptr(),
                     st.cuda_stream)
        zi[j].copy_(zb[j])  # AsymQuantizer's zeros_x.to(torch.int8)

    def gemm(i):
        j = i % len(xs)
        _native.call("srq_w4a4_linear_asym", qb[j].data_ptr(), sb[j].data_ptr(),
                     zi[j].data_ptr(), wts[i % nsets].data_ptr(), wsc.data_ptr(),
                     wsum[i % nsets].data_ptr(), None, M, N, K, ob[j].data_ptr(),
                     st.cuda_stream)

    def both(i):
        had(i)
        gemm(i)

    n = max(20, min(nsets, 64))
    t_all = _time_launches(both, n, st) * 1e3
    t_had = _time_launches(had, n, st) * 1e3
    t_gemm = _time_launches(gemm, n, st) * 1e3
    ops = 2.0 * M * N * K
    res = {"M": M, "K": K, "N": N, "hadamard": f"had_{k} x H_{K // k}", "weight_sets": nsets,
           "qlinear": _roof(t_all, ops, M * K * 2 + N * K // 2 + M * N * 2 + M * 4 + N * 6),
           "had_sign_asym_quant": _roof(t_had, 0.0, M * K * 2 + M * K // 2 + M * 4),
           "w4a4_linear_asym": _roof(t_gemm, ops, M * K // 2 + N * K // 2 + M * N * 2 + M * 3
                                     + N * 6)}
    del xs, wts, qb, sb, zb, zi, ob
    torch.cuda.empty_cache()
    return res


def bench_qlinear_bf6(dev, M, K, N, seed, n_out=8, mag=50.0, min_bytes=2.2e9, reps=20):
    """The cfg2 QLinear on the opt-in bf6 path: had_sign_quant_bf6 (rotation +
    sign + int4 quantizer writing the codes in the bf6 block layout) and
    w4a4_linear_bf6 (the int4 codes as exact e3m2 values on the 6-bit-operand
    MFMA, weights converted once with i4_to_bf6).  Bit-identical to the int8
    path (checked here on the first set); its GEMM is priced against the
    fp6 MFMA peak it runs on."""
    from signrot_amd import _CUDA
    from signrot_amd.functional.hadamard import get_hadK
    g = torch.Generator(device=dev).manual_seed(seed)
    had, k = get_hadK(K)
    hadk = had.half().to(dev).contiguous()
    sign = (torch.randint(0, 2, (K,), device=dev, generator=g).to(torch.int8) * 2 - 1)
    set_bytes = M * K * 2 + _CUDA.bf6_bytes(N, K) + _CUDA.bf6_bytes(M, K) + M * N * 2
    nsets = max(1, min(64, math.ceil(min_bytes / set_bytes)))
    x0 = torch.randn(M, K, device=dev, generator=g)
    ch = torch.randperm(K, device=dev, generator=g)[:n_out]
    x0[:, ch] *= mag
    x0 = x0.half()
    xs = [x0] + [x0.clone() for _ in range(min(nsets, 8) - 1)]
    w4 = _rand_w(N, K, dev, g)
    ws6 = [_CUDA.i4_to_bf6(w4) for _ in range(nsets)]
    wsc = (torch.rand(N, device=dev, generator=g) * 1e-3 + 1e-4).half()
    q6s = [_CUDA.had_sign_quant_bf6(x, hadk, k, sign) for x in xs]
    q4, s4 = _CUDA.had_sign_quant(x0, hadk, k, sign)
    ref = _CUDA.w4a4_linear(q4, s4.view(-1), w4, wsc)
    got = _CUDA.w4a4_linear_bf6(q6s[0][0], q6s[0][1].view(-1), ws6[0], wsc, M, N, K)
    assert torch.equal(got, ref), "bf6 path differs from the int8 path"
    del w4, q4, s4, ref, got

    def had(i):
        return _CUDA.had_sign_quant_bf6(xs[i % len(xs)], hadk, k, sign)

    def gemm(i):
        q6, sc = q6s[i % len(xs)]
        return _CUDA.w4a4_linear_bf6(q6, sc.view(-1), ws6[i % nsets], wsc, M, N, K)

    def both(i):
        q6, sc = had(i)
        return _CUDA.w4a4_linear_bf6(q6, sc.view(-1), ws6[i % nsets], wsc, M, N, K)

    n = max(reps, min(nsets, 64))
    t_all = _time_graph(both, n) * 1e3
    t_had = _time_graph(had, n) * 1e3
    t_gemm = _time_graph(gemm, n) * 1e3
    ops = 2.0 * M * N * K
    gemm_line = _roof(t_gemm, ops, _CUDA.bf6_bytes(M, K) + _CUDA.bf6_bytes(N, K) + M * N * 2)
    gemm_line["frac_mfma_fp6"] = round(gemm_line["TOPS"] / PEAK_FP6_TOPS, 4)
    res = {"M": M, "K": K, "N": N, "hadamard": f"had_{k} x H_{K // k}", "weight_sets": nsets,
           "timing": "hip_graph",
           "qlinear": _roof(t_all, ops, M * K * 2 + _CUDA.bf6_bytes(N, K) + M * N * 2),
           "had_sign_quant_bf6": _roof(t_had, 0.0, M * K * 2 + _CUDA.bf6_bytes(M, K) + M * 2),
           "w4a4_linear_bf6": gemm_line}
    del xs, ws6, q6s
    torch.cuda.empty_cache()
    return res


def bench_mlp70b(dev, M, seed, hidden=8192, ffn=28672, reps=10, min_bytes=2.2e9):
    """Config 4: Llama-3-70B-shape W4A4 MLP block: per-token int4 quant of x,
    the gate and up W4A4 linears as one GEMM over their rows interleaved in
    blocks of 8 with the SwiGLU in its epilogue (the decode layer's layout),
    had_28 x H_1024 rotation + sign + quant in one launch, down W4A4
    linear."""
    from signrot_amd import _CUDA
    from signrot_amd.functional.hadamard import get_hadK
    g = torch.Generator(device=dev).manual_seed(seed)
    had, k = get_hadK(ffn)
    hadk = had.half().to(dev).contiguous()
    sign = (torch.randint(0, 2, (ffn,), device=dev, generator=g).to(torch.int8) * 2 - 1)
    wbytes = 3 * ffn * hidden // 2
    nsets = max(1, math.ceil(min_bytes / wbytes))
    Wgu = [_rand_w(2 * ffn, hidden, dev, g) for _ in range(nsets)]
    Wd = [_rand_w(hidden, ffn, dev, g) for _ in range(nsets)]
    sgu = torch.full((2 * ffn,), 1.0 / hidden, dtype=torch.float16, device=dev)
    # weight preparation (once, untimed): gate/up rows in blocks of 8
    il = [_CUDA.interleave_gate_up(w, sgu, ffn) for w in Wgu]
    del Wgu
    sd = torch.full((hidden,), 1.0 / ffn, dtype=torch.float16, device=dev)
    x = torch.randn(M, hidden, device=dev, generator=g)
    ch = torch.randperm(hidden, device=dev, generator=g)[:8]
    x[:, ch] *= 100.0
    x = x.half()

    def mlp(i):
        j = i % nsets
        q, s = _CUDA.sym_quant_dynamic(x)
        a = _CUDA.w4a4_linear_swiglu(q, s.view(-1), il[j][0], il[j][1])
        qd, sdn = _CUDA.had_sign_quant(a, hadk, k, sign)
        return _CUDA.w4a4_linear(qd, sdn.view(-1), Wd[j], sd)

    st = torch.cuda.current_stream()
    t_eager = _time_launches(mlp, max(reps, nsets), st) * 1e3
    t = _time_graph(mlp, max(reps, nsets)) * 1e3
    ops = 2.0 * M * 3 * hidden * ffn
    nbytes = wbytes + M * hidden * 2 * 2
    del il, Wd
    torch.cuda.empty_cache()
    return {"M": M, "hidden": hidden, "ffn": ffn, "hadamard": f"had_{k} x H_{ffn // k}",
            "weight_sets": nsets, "timing": "hip_graph", "mlp_eager_us": round(t_eager, 2),
            "mlp": _roof(t, ops, nbytes)}


def bench_moe(dev, seed, tokens=512, hidden=4096, ffn=14336, experts=8, top_k=2, reps=10):
    """Config 5: Mixtral-8x7B-shape W4A4 MoE FFN (SignRotMoEBlock, grouped
    path): 8 experts, top-2 routing of 512 tokens (router logits N(0,1)
    seeded through a random router), hidden 4096, FFN 14336, SwiGLU,
    had_28 x H_512 + per-expert sign on the down-proj input.  The block has
    no host synchronization, so it is timed as HIP-graph replays (the eager
    time, which adds the module's host work between launches, beside it)."""
    from signrot_amd.nn import SignRotMoEBlock
    g = torch.Generator(device=dev).manual_seed(seed)
    gate = torch.nn.Linear(hidden, experts, bias=False, dtype=torch.float16, device=dev)
    with torch.no_grad():
        gate.weight.normal_(0, 1.0 / math.sqrt(hidden), generator=g)

    def w(n, k):
        return torch.randint(0, 256, (experts, n, k // 2), dtype=torch.uint8, device=dev,
                             generator=g)

    def sc(n, k):
        return torch.full((experts, n), 1.0 / k, dtype=torch.float16, device=dev)

    sign = torch.randint(0, 2, (experts, ffn), dtype=torch.int8, device=dev, generator=g) * 2 - 1
    blk = SignRotMoEBlock(gate, top_k=top_k, norm_topk_prob=True, w_gate=w(ffn, hidden),
                          s_gate=sc(ffn, hidden), w_up=w(ffn, hidden), s_up=sc(ffn, hidden),
                          w_down=w(hidden, ffn), s_down=sc(hidden, ffn), sign_down=sign).eval()
    xs = [torch.randn(1, tokens, hidden, device=dev, generator=g).half() for _ in range(4)]
    st = torch.cuda.current_stream()
    with torch.no_grad():
        t_eager = _time_launches(lambda i: blk(xs[i % len(xs)]), reps, st) * 1e3
        t = _time_graph(lambda i: blk(xs[i % len(xs)]), reps) * 1e3
        counts = blk.route(xs[0].view(-1, hidden)).counts
    rows = tokens * top_k
    ops = 2.0 * rows * 3 * hidden * ffn
    nbytes = 3 * experts * ffn * hidden // 2
    res = {"tokens": tokens, "experts": experts, "top_k": top_k, "hidden": hidden, "ffn": ffn,
           "rows_per_expert": counts.tolist(), "timing": "hip_graph",
           "block_eager_us": round(t_eager, 2), "block": _roof(t, ops, nbytes)}
    del blk, xs
    torch.cuda.empty_cache()
    return res


def bench_prefill_attention(dev, B, T, Hq, Hkv, seed, reps=20):
    """Prefill attention of the layer's first update (the flash-attn 2 call
    it replaces): causal GQA over fp16 q/k/v [B, T, H, 128].  Work is the
    causal half of QK^T and PV: 4 * B * Hq * 128 * T (T + 1) / 2 flops."""
    from signrot_amd import _CUDA
    st = torch.cuda.current_stream()
    g = torch.Generator(device=dev).manual_seed(seed)
    q = torch.randn(B, T, Hq, 128, device=dev, generator=g).half()
    k = torch.randn(B, T, Hkv, 128, device=dev, generator=g).half()
    v = torch.randn(B, T, Hkv, 128, device=dev, generator=g).half()
    t = _time_launches(lambda i: _CUDA.prefill_attention(q, k, v), reps, st) * 1e3
    flops = 4.0 * B * Hq * 128 * T * (T + 1) / 2
    res = {"B": B, "T": T, "Hq": Hq, "Hkv": Hkv, "us": round(t, 2),
           "TFLOP/s": round(flops / t * 1e-6, 1),
           "mfma_frac_f16": round(flops / t * 1e-6 / 2500.0, 4)}
    del q, k, v
    torch.cuda.empty_cache()
    return res


def bench_configs(args, dev):
    """The benchmark configs other than the headline one, each at its own
    shape (cfg1 q_proj at M=16, the cfg2 M sweep, the cfg4 70B MLP, the cfg5
    MoE block), the cfg2
    QLinear with asymmetric activations and on the opt-in bf6 path, and the
    prefill attention (Llama-70B heads)."""
    out = {"cfg1_qproj_M16": bench_qlinear(dev, 16, 4096, 4096, args.seed + 10, n_out=4,
                                           mag=100.0),
           "cfg2_sweep": [bench_qlinear(dev, m, 14336, 4096, args.seed + 20 + m)
                          for m in (1, 16, 128, 2048, 8192)],
           "cfg2_asym_M2048": bench_qlinear_asym(dev, 2048, 14336, 4096, args.seed + 25),
           "cfg2_bf6_M2048": bench_qlinear_bf6(dev, 2048, 14336, 4096, args.seed + 26),
           "cfg4_mlp70b": [bench_mlp70b(dev, m, args.seed + 30 + m) for m in (1, 32, 512, 4096)],
           "cfg5_moe": bench_moe(dev, args.seed + 40),
           "prefill_attention": [bench_prefill_attention(dev, 1, t, 64, 8, args.seed + 50 + t)
                                 for t in (512, 2048, 8192)]}
    return out


def measured_traffic(kernel, M, K, N):
    """HBM bytes per launch of `kernel` at this shape from the committed
    rocprofv3 FETCH_SIZE / WRITE_SIZE passes (profiles/traffic_cfg2.json,
    already scaled by the plain-copy calibration), or None."""
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles",
                        "traffic_cfg2.json")
    try:
        with open(path) as f:
            rec = json.load(f)
    except (OSError, ValueError):
        return None
    entry = rec.get("kernels", {}).get(kernel)
    if not entry or [rec.get("M"), rec.get("K"), rec.get("N")] != [M, K, N]:
        return None
    return entry.get("hbm_bytes")


def traffic_commit():
    """The commit the committed traffic figures were measured at."""
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles",
                        "traffic_cfg2.json")
    try:
        with open(path) as f:
            return json.load(f).get("measured_at")
    except (OSError, ValueError):
        return None


def gemm_kernel_name(M, N, K=None, split=False):
    """Kernel srq_w4a4_linear(_ws) launches for M x N outputs (gemm.hip
    dispatch, fp16 output)."""
    def cdiv(a, b):
        return -(-a // b)
    if M <= 32:
        return "gemm_stream_kernel (srq_w4a4_linear)"
    if M <= 64:
        return "gemm_skinny_kernel (srq_w4a4_linear)"
    if M >= 1024 and cdiv(M, 256) * cdiv(N, 256) >= 256:
        return "gemm_sq_kernel (srq_w4a4_linear, 256 x 256 tiles)"
    if split:
        return "gemm_grouped_kernel split-K form + splitk_reduce_kernel (srq_w4a4_linear_ws)"
    if M < 1024 and cdiv(M, 128) * cdiv(N, 128) >= 192 and cdiv(M, 256) * cdiv(N, 128) < 512:
        return "gemm_grouped_kernel dense form (srq_w4a4_linear, 128 x 128 tiles)"
    if M >= 1024 or cdiv(M, 256) * cdiv(N, 128) >= 512:
        return "gemm_big_kernel (srq_w4a4_linear, 256 x 128 tiles)"
    return "gemm_ring_kernel (srq_w4a4_linear)"


def calibrate_copy(dev, reps=3):
    """`reps` launches of torch's device copy over COPY_BYTES bytes: each
    reads and writes exactly COPY_BYTES, so FETCH_SIZE / WRITE_SIZE per
    dispatch divided by COPY_BYTES is the counters' scale factor."""
    src = torch.randint(0, 255, (COPY_BYTES // 4,), dtype=torch.int32, device=dev)
    dst = torch.empty_like(src)
    for _ in range(reps):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"calibrate_copy_bytes": COPY_BYTES, "reps": reps}), flush=True)


def profile_workloads(args, dev):
    """One workload of the committed rocprofv3 summaries, a few launches
    over weight sets that exceed the MALL."""
    t0 = time.perf_counter()
    name = args.profile
    if name.startswith("cfg2_M"):
        m = int(name[len("cfg2_M"):])
        res = bench_qlinear(dev, m, 14336, 4096, args.seed + 20 + m, reps=5, min_bytes=6e8)
    elif name == "cfg4_M512":
        res = bench_mlp70b(dev, 512, args.seed + 30 + 512, reps=3, min_bytes=6e8)
    elif name == "cfg5_moe":
        res = bench_moe(dev, args.seed + 40, reps=3)
    elif name == "prefill_T8192":
        res = bench_prefill_attention(dev, 1, 8192, 64, 8, args.seed + 50 + 8192, reps=3)
    elif name == "cfg2_bf6_M2048":
        res = bench_qlinear_bf6(dev, 2048, 14336, 4096, args.seed + 26, reps=5, min_bytes=6e8)
    else:
        args.decode_steps, args.decode_layers = 3, 2
        res = bench_decode_layer(args, dev)
    print(json.dumps({"profile": name, "result": res,
                      "wall_s": round(time.perf_counter() - t0, 1)}), flush=True)


def cpu_model():
    """The host CPU's model name (from /proc/cpuinfo), or None."""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return None


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU only (got --gpus {args.gpus}); "
              "the multi-GPU sharding is a design note, not a measured path", file=sys.stderr)
        sys.exit(2)
    if not torch.cuda.is_available():
        print("bench.py: no GPU visible", file=sys.stderr)
        sys.exit(1)
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    if args.prefill_attention_only:
        for t in (512, 2048, 8192):
            print(json.dumps(bench_prefill_attention(dev, 1, t, 64, 8, args.seed + 50 + t)),
                  flush=True)
        return
    if args.calibrate_copy:
        calibrate_copy(dev)
        return
    if args.profile:
        profile_workloads(args, dev)
        return
    from signrot_amd import _CUDA

    M, K, N = args.M, args.K, args.N
    x0, hadk, k, sign, wq0, ws, wfq = make_inputs(args, dev)
    set_bytes = x0.numel() * 2 + wq0.numel() + M * K // 2 + M * N * 2
    nsets = max(1, math.ceil(args.min_bytes / set_bytes))
    xs = [x0] + [x0.clone() for _ in range(nsets - 1)]
    wqs = [wq0] + [wq0.clone() for _ in range(nsets - 1)]
    qbufs = [torch.empty(M, K // 2, dtype=torch.uint8, device=dev) for _ in range(nsets)]
    sbufs = [torch.empty(M, 1, dtype=torch.float16, device=dev) for _ in range(nsets)]
    outs = [torch.empty(M, N, dtype=torch.float16, device=dev) for _ in range(nsets)]

    from signrot_amd import _native

    stream = torch.cuda.current_stream()

    def step(i):
        # on the current stream at call time (the capture stream under
        # graph capture)
        j = i % nsets
        cs = torch.cuda.current_stream().cuda_stream
        _native.call("srq_had_sign_quant", xs[j].data_ptr(), M, K, k,
                     hadk.data_ptr() if hadk is not None else None, sign.data_ptr(), 0, 1.0,
                     qbufs[j].data_ptr(), sbufs[j].data_ptr(), cs)
        _native.call("srq_w4a4_linear", qbufs[j].data_ptr(), sbufs[j].data_ptr(),
                     wqs[j].data_ptr(), ws.data_ptr(), None, M, N, K, outs[j].data_ptr(), cs)

    # correctness guard on the measured buffers: fused path == module path
    from signrot_amd.functional import kernel
    q_ref, s_ref = kernel.had_sign_quant(x0, hadk, k, sign)
    step(0)
    torch.cuda.synchronize()
    assert torch.equal(qbufs[0], q_ref) and torch.equal(sbufs[0], s_ref)

    for i in range(args.warmup):
        step(i)
    torch.cuda.synchronize()

    # eager: the K steps launched one call at a time (reported beside the
    # timed figure)
    t_start = torch.cuda.Event(enable_timing=True)
    t_stop = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t_start.record(stream)
    for i in range(args.steps):
        step(i)
    t_stop.record(stream)
    torch.cuda.synchronize()
    ms_step_eager = t_start.elapsed_time(t_stop) / args.steps

    # timed: the K steps captured once into a HIP graph (as a serving loop
    # runs them, without the host's per-launch cost between kernels),
    # replayed once untimed, then exactly once between HIP events
    side = torch.cuda.Stream()
    side.wait_stream(stream)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=side):
        for i in range(args.steps):
            step(i)
    graph.replay()
    torch.cuda.synchronize()
    t_start.record(stream)
    graph.replay()
    t_stop.record(stream)
    torch.cuda.synchronize()
    ms_step = t_start.elapsed_time(t_stop) / args.steps
    del graph
    # the replayed graph computed what the eager steps did
    assert torch.equal(qbufs[0], q_ref) and torch.equal(sbufs[0], s_ref)

    # per-kernel averages: each kernel alone, back to back, over the same
    # rotating buffers, HIP events on the launch stream around the loop
    def time_kernel(launch):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        e0.record(stream)
        for i in range(args.steps):
            launch(i % nsets)
        e1.record(stream)
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / args.steps

    had_ms = time_kernel(lambda j: _native.call(
        "srq_had_sign_quant", xs[j].data_ptr(), M, K, k,
        hadk.data_ptr() if hadk is not None else None, sign.data_ptr(), 0, 1.0,
        qbufs[j].data_ptr(), sbufs[j].data_ptr(), stream.cuda_stream))
    gemm_ms = time_kernel(lambda j: _native.call(
        "srq_w4a4_linear", qbufs[j].data_ptr(), sbufs[j].data_ptr(), wqs[j].data_ptr(),
        ws.data_ptr(), None, M, N, K, outs[j].data_ptr(), stream.cuda_stream))

    ops = 2.0 * M * N * K
    value = ops / (ms_step * 1e-3) / 1e12
    gemm_tops = ops / (gemm_ms * 1e-3) / 1e12
    had_bytes = M * K * 2 + M * K // 2 + M * 2 + K + (k * k * 2 if k > 1 else 0)
    had_gbs = had_bytes / (had_ms * 1e-3) / 1e9
    gemm_bytes = M * K // 2 + N * K // 2 + M * 2 + N * 2 + M * N * 2

    decode = None
    if not args.no_decode:
        del xs, wqs, qbufs, outs
        torch.cuda.empty_cache()
        decode = bench_decode_layer(args, dev)

    configs = None
    if not args.no_configs:
        configs = bench_configs(args, dev)

    cpu = None
    if not args.no_cpu_baseline:
        cpu = time_cpu_baseline(args, x0, hadk, k, sign, wfq)

    line = {
        "metric": METRIC,
        "value": round(value, 2),
        "unit": "TOPS",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 5),
        "timing": "hip_graph",
        "ms_per_step_eager": round(ms_step_eager, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int4",
        "data": "synthetic",
        "config": {"workload": (f"cfg2 Llama-3-8B down_proj W4A4 QLinear prefill: "
                                f"had_{k} x H_{K // k} rotation + SignRot sign + per-token "
                                f"int4 act-quant + int4 GEMM + fp16 dequant"),
                   "M": M, "K": K, "N": N, "input_sets": nsets},
        "roofline": {"bound": "mfma", "achieved": round(gemm_tops, 1),
                     "peak": PEAK_INT8_TOPS, "unit": "TFLOP/s",
                     "frac": round(gemm_tops / PEAK_INT8_TOPS, 4),
                     "traffic": measured_traffic(gemm_kernel_name(M, N).split()[0], M, K, N),
                     "traffic_measured_at": traffic_commit(),
                     "kernel": gemm_kernel_name(M, N),
                     "algorithmic_ops": ops, "avg_launch_us": round(gemm_ms * 1e3, 2)},
        "kernels": {
            "had_sign_quant": {"avg_us": round(had_ms * 1e3, 2), "bound": "hbm",
                               "algorithmic_bytes": had_bytes,
                               "achieved_GBs": round(had_gbs, 1),
                               "frac_hbm": round(had_gbs / PEAK_HBM_GBS, 4),
                               "traffic": measured_traffic("had512_mfma_kernel<4, 1, false, 1>", M, K, N)},
            "w4a4_linear": {"avg_us": round(gemm_ms * 1e3, 2), "bound": "mfma",
                            "algorithmic_bytes": gemm_bytes,
                            "achieved_TOPS": round(gemm_tops, 1),
                            "frac_mfma": round(gemm_tops / PEAK_INT8_TOPS, 4)},
        },
        "decode_layer": decode,
        "configs": configs,
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
