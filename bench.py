"""Benchmark of the HiF8 fake-quant linear path on one MI355X.

Workload (Wan-14B 720P): one HIF8Linear forward of the FFN-up
projection, x [75600, 5120] bf16 (N(0,1), 16 outlier channels x20) against
W [13824, 5120] held as packed 8-bit HiF8 codes (N(0,0.02), prepacked once,
outside the timed region).  A step = amax+scale of x, fake-quant of x, the GEMM of
x_q and the dequantised weight + bias -> y [75600, 13824] bf16: the reference's
_HIF8LinearFunction.forward (ospnext/modules/hif8_linear.py:68-86).

value = 2*M*N*K / step time (TFLOP/s).  At this M the step takes HIF8Linear's decode-once
route (the weight codes decoded to bf16 once per call, then the decode-free GEMM); the fused
dequant-GEMM route is timed beside it (other_route).  The per-kernel times come from HIP
events on the stream the kernels run on (torch's current stream).

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu]
                    [--route auto|fused|decode_once] [--shapes ...]
"""
from __future__ import annotations

import argparse
import json
import os
import platform
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
METRIC = "HiF8 linear TFLOP/s + encode GB/s (14B 720P shapes), 1 GPU, % of roofline"
PEAK_BF16_TFLOPS = 2500.0   # MI355X dense bf16 MFMA
PEAK_HBM_GBPS = 8000.0      # MI355X HBM3E


def log(msg):
    print(msg, file=sys.stderr, flush=True)


def make_inputs(torch, M, K, N, seed=0, dev="cuda:0", outlier_channels=16):
    g = torch.Generator(device=dev).manual_seed(seed)
    x = torch.randn(M, K, generator=g, device=dev, dtype=torch.float32)
    ch = torch.randperm(K, generator=g, device=dev)[:outlier_channels]
    x[:, ch] *= 20
    x = x.to(torch.bfloat16)
    w = (torch.randn(N, K, generator=g, device=dev, dtype=torch.float32) * 0.02).to(torch.bfloat16)
    b = torch.zeros(N, dtype=torch.bfloat16, device=dev)
    return x, w, b


def time_linear(pkg, torch, x, packed, b, steps, warmup, route="fused"):
    """Times steps of [amax+scale, quantise, GEMM]; returns per-phase ms lists.

    route "fused": the fused dequant-GEMM hif8_linear_fwd on the packed weight codes;
    "decode_once": the GEMM phase is hif8_decode of the weight codes into a bf16 buffer, then the
    decode-free GEMM hif8_linear_fwd_wq (the HIF8Linear route where hif8_linear.decode_once(M, K));
    its two parts are timed separately as well."""
    st = pkg.QuantState(x.device)
    L = pkg._lib.load()
    stream = pkg._lib.stream_ptr(x.device)
    M, K = x.shape
    N = packed.shape[0]
    y = torch.empty(M, N, dtype=torch.bfloat16, device=x.device)
    a = torch.empty((M, K), dtype=torch.bfloat16, device=x.device)
    wq = torch.empty((N, K), dtype=torch.bfloat16, device=x.device) if route == "decode_once" else None

    def amax():
        pkg._lib.check(L.hif8_absmax_scale(x.data_ptr(), 0, x.numel(), 15.0, st.ptr, stream), "amax")

    def quant():
        pkg._lib.check(L.hif8_fake_quant(x.data_ptr(), 0, x.numel(), st.ptr, a.data_ptr(), 0, stream), "qdq")

    def wdecode():
        pkg._lib.check(L.hif8_decode(packed.codes.data_ptr(), N * K, packed.state.ptr, 0, wq.data_ptr(), stream),
                       "decode")

    def gemm():
        if route == "decode_once":
            pkg._lib.check(L.hif8_linear_fwd_wq(a.data_ptr(), wq.data_ptr(), b.data_ptr(), y.data_ptr(), M, N, K,
                                                stream), "linear_wq")
        else:
            pkg._lib.check(L.hif8_linear_fwd(a.data_ptr(), packed.codes.data_ptr(), packed.state.ptr, b.data_ptr(),
                                             y.data_ptr(), M, N, K, stream), "linear")

    def wdec_maybe():
        if route == "decode_once":
            wdecode()

    for _ in range(warmup):
        amax(); quant(); wdec_maybe(); gemm()
    torch.cuda.synchronize()
    ev = [[torch.cuda.Event(enable_timing=True) for _ in range(5)] for _ in range(steps)]
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(steps):
        e = ev[i]
        e[0].record()
        amax()
        e[1].record()
        quant()
        e[2].record()
        wdec_maybe()
        e[3].record()
        gemm()
        e[4].record()
    torch.cuda.synchronize()
    wall = (time.perf_counter() - t0) * 1e3
    return {"wall_ms": wall, "amax": [e[0].elapsed_time(e[1]) for e in ev],
            "quant": [e[1].elapsed_time(e[2]) for e in ev], "wdecode": [e[2].elapsed_time(e[3]) for e in ev],
            "gemm": [e[3].elapsed_time(e[4]) for e in ev], "y": y}


TRAFFIC_DOC = os.path.join(ROOT, "profiles", "hif8_kernels_14b_720p_hbm_traffic.md")


def measured_traffic(kernel: str):
    """HBM-side bytes per launch of `kernel` at the 14B FFN-up shape, as recorded from the two
    rocprofv3 PMC passes (FETCH_SIZE, WRITE_SIZE) whose commands and calibration the summary
    file gives; None if the summary has no figure for it."""
    try:
        with open(TRAFFIC_DOC) as f:
            for line in f:
                if line.startswith(f"traffic_bytes_per_launch {kernel}:"):
                    return int(line.split(":")[1])
    except OSError:
        pass
    return None


def time_ffn(pkg, torch, x, reps):
    """The 14B FFN (osp_next.py:873-877) on x: HIF8FFN's fused route (the up-projection's epilogue
    folds the GELU statistic, the down-projection's quantisation applies GELU) against the plain
    sequence HIF8Linear -> GELU -> HIF8Linear; and the up-projection's GEMM with and without the
    GELU-statistic epilogue on the same operands (k_linear_w16<1> against <0>), with the down
    input's quantisation with GELU (hif8_gelu_fake_quant) against the plain fake quant of the
    same tensor."""
    dim, ffn = x.shape[1], 13824
    torch.manual_seed(3)
    mod = pkg.HIF8FFN(dim, ffn, device=x.device, dtype=torch.bfloat16)
    with torch.no_grad():
        for p in mod.parameters():
            p.normal_(0, 0.02)
    mod[0].prepack(drop_weight=False)
    mod[2].prepack(drop_weight=False)
    out = {}

    def timed(fn, n):
        for _ in range(2):
            fn()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(n):
            fn()
        e1.record()
        torch.cuda.synchronize()
        return round(e0.elapsed_time(e1) / n, 4)

    def timed_pair(fa, fb, n):
        for _ in range(2):
            fa()
            fb()
        torch.cuda.synchronize()
        blocks = max(2, n // 2)
        ev = [[torch.cuda.Event(enable_timing=True) for _ in range(4)] for _ in range(blocks)]
        per = max(1, n // blocks)
        for e in ev:
            e[0].record()
            for _ in range(per):
                fa()
            e[1].record()
            e[2].record()
            for _ in range(per):
                fb()
            e[3].record()
        torch.cuda.synchronize()
        ta = sum(e[0].elapsed_time(e[1]) for e in ev) / (blocks * per)
        tb = sum(e[2].elapsed_time(e[3]) for e in ev) / (blocks * per)
        return round(ta, 4), round(tb, 4)

    with torch.no_grad():
        out["fused_ms"] = timed(lambda: mod(x), reps)
        out["sequence_ms"] = timed(lambda: torch.nn.Sequential.forward(mod, x), reps)
        a, _, _ = pkg.quantize_activation(x, 15.0, "bf16")
        w_q = mod[0]._packed_weight().dequantize()
        st = pkg.QuantState(x.device)
        # The two GEMMs alternate in short blocks, so that the clock's drift under sustained load
        # (the kernels run at the board's power limit) falls on both alike.
        out["up_gemm_plain_ms"], out["up_gemm_gelu_stat_ms"] = timed_pair(
            lambda: pkg.linear_fwd_wq(a, w_q, mod[0].bias),
            lambda: pkg.linear_fwd_wq(a, w_q, mod[0].bias, st, 15.0), reps)
        y = pkg.linear_fwd_wq(a, w_q, mod[0].bias, st, 15.0)
        out["gelu_fake_quant_ms"] = timed(lambda: pkg.gelu_fake_quant(y, st, 15.0), reps)
        st2 = pkg.absmax_scale(y, 15.0, pkg.QuantState(x.device))
        out["plain_fake_quant_ms"] = timed(lambda: pkg.fake_quant(y, st2), reps)
        del a, w_q, y
    flops = 2.0 * 2 * x.shape[0] * dim * ffn
    out["fused_TFLOPs"] = round(flops / (out["fused_ms"] * 1e-3) / 1e12, 1)
    out["speedup"] = round(out["sequence_ms"] / out["fused_ms"], 4)
    out["up_epilogue_cost"] = round(out["up_gemm_gelu_stat_ms"] / out["up_gemm_plain_ms"] - 1.0, 4)
    # the GELU quantisation pass reads y and writes x_q: 2 + 2 bytes per element (its one-workgroup
    # prep kernel, which tables x_q over y for the state, is inside the timed call)
    qbytes = 4.0 * x.shape[0] * ffn
    out["gelu_fake_quant_GBps"] = round(qbytes / (out["gelu_fake_quant_ms"] * 1e-3) / 1e9, 1)
    out["gelu_fake_quant_frac"] = round(out["gelu_fake_quant_GBps"] / 8000.0, 4)
    out["plain_fake_quant_GBps"] = round(qbytes / (out["plain_fake_quant_ms"] * 1e-3) / 1e9, 1)
    out["what"] = "FFN 5120->13824->5120 on x[75600,5120] bf16, prepacked weights, no autograd"
    del mod
    return out


def time_module_graph(pkg, torch, M, reps):
    """HIF8Linear.forward (prepacked, no autograd) on the 1.3B 480P shapes, called eagerly and
    replayed from a HIP graph (torch.cuda.CUDAGraph) that captured the same call: at these sizes
    the four launches of a step (amax, fake quant, weight decode, GEMM) and their host-side
    overhead are a visible part of it."""
    out = {}
    for name, n_, k_, seed in (("qkvo", 1536, 1536, 2), ("ffn_up", 8960, 1536, 3), ("ffn_down", 1536, 8960, 4)):
        x, _, _ = make_inputs(torch, M, k_, n_, seed=seed, outlier_channels=8)
        torch.manual_seed(seed)
        lin = pkg.HIF8Linear(k_, n_, bias=True, device=x.device, dtype=torch.bfloat16)
        with torch.no_grad():
            lin.weight.normal_(0, 0.02)
            lin.bias.zero_()
            lin.prepack()
            side = torch.cuda.Stream()
            side.wait_stream(torch.cuda.current_stream())
            with torch.cuda.stream(side):
                for _ in range(2):
                    lin(x)
            torch.cuda.current_stream().wait_stream(side)
            torch.cuda.synchronize()
            graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(graph):
                lin(x)
            res = {}
            for label, fn in (("eager_ms", lambda: lin(x)), ("graph_ms", graph.replay)):
                for _ in range(3):
                    fn()
                torch.cuda.synchronize()
                e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                e0.record()
                for _ in range(reps):
                    fn()
                e1.record()
                torch.cuda.synchronize()
                res[label] = round(e0.elapsed_time(e1) / reps, 4)
            res["graph_TFLOPs"] = round(2.0 * M * n_ * k_ / (res["graph_ms"] * 1e-3) / 1e12, 1)
            out[name] = res
            del graph
        del lin, x
    return out


def time_backward(pkg, torch, x, packed, reps):
    """The backward of the FFN-up HIF8Linear (hif8_linear.py:88-111) at the 14B 720P shape: the
    gradient's _quant with scale_max 224, dgrad grad_q [M, N] @ w_q [N, K] (the transposed codes
    decoded once, then the decode-free GEMM) and wgrad grad_q^T @ x_q (hif8_linear_wgrad: the
    decode-free GEMM reading both operands token-major with transposing LDS loads, its last
    partial wave split over token ranges); for comparison the GEMMs without the split and wgrad's
    transposed route (both operands transposed, then the row-major GEMM); each phase timed with HIP
    events on the launch stream.  hipBLASLt on the same operands for context."""
    dev = x.device
    M, K = x.shape
    N = packed.shape[0]
    L = pkg._lib.load()
    stream = pkg._lib.stream_ptr(dev)
    gen = torch.Generator(device=dev).manual_seed(6)
    gy = (torch.randn(M, N, generator=gen, device=dev) * 1e-3).to(torch.bfloat16)
    xq = pkg.fake_quant(x, pkg.absmax_scale(x, 15.0, pkg.QuantState(dev)))
    st = pkg.QuantState(dev)
    gq = torch.empty_like(gy)
    codes_t = packed.codes_t()
    w_qt = torch.empty((K, N), dtype=torch.bfloat16, device=dev)
    Mp = (M + 63) // 64 * 64
    g_t = torch.empty((N, Mp), dtype=torch.bfloat16, device=dev)
    x_t = torch.empty((K, Mp), dtype=torch.bfloat16, device=dev)
    gx = torch.empty((M, K), dtype=torch.bfloat16, device=dev)
    gw = torch.empty((N, K), dtype=torch.bfloat16, device=dev)
    ws_bytes = int(L.hif8_linear_split_workspace_bytes(N, K, M))
    ws = torch.empty(max(ws_bytes // 4, 1), dtype=torch.float32, device=dev)
    ws_d_bytes = int(L.hif8_linear_split_workspace_bytes(M, K, N))
    ws_d = torch.empty(max(ws_d_bytes // 4, 1), dtype=torch.float32, device=dev)
    ck = pkg._lib.check
    phases = {
        "grad_quant": lambda: (ck(L.hif8_absmax_scale(gy.data_ptr(), 0, gy.numel(), 224.0, st.ptr, stream), "amax"),
                               ck(L.hif8_fake_quant(gy.data_ptr(), 0, gy.numel(), st.ptr, gq.data_ptr(), 0, stream),
                                  "qdq")),
        "dgrad_wdecode": lambda: ck(L.hif8_decode(codes_t.data_ptr(), N * K, packed.state.ptr, 0, w_qt.data_ptr(),
                                                  stream), "decode"),
        "dgrad_gemm": lambda: ck(L.hif8_linear_fwd_wq_split(gq.data_ptr(), w_qt.data_ptr(), None, gx.data_ptr(), M,
                                                            K, N, ws_d.data_ptr(), ws_d_bytes, stream), "dgrad"),
        "dgrad_gemm_unsplit": lambda: ck(L.hif8_linear_fwd_wq(gq.data_ptr(), w_qt.data_ptr(), None, gx.data_ptr(), M,
                                                              K, N, stream), "dgrad whole"),
        "wgrad_gemm": lambda: ck(L.hif8_linear_wgrad(gq.data_ptr(), xq.data_ptr(), gw.data_ptr(), M, N, K,
                                                     ws.data_ptr(), ws_bytes, stream), "wgrad"),
        # for comparison: every tile computed whole (no split tail) ...
        "wgrad_gemm_unsplit": lambda: ck(L.hif8_linear_wgrad(gq.data_ptr(), xq.data_ptr(), gw.data_ptr(), M, N, K,
                                                             None, 0, stream), "wgrad whole"),
        # ... and the transposed route: both operands transposed, then the row-major GEMM
        "wgrad_transposed_transposes": lambda: (
            ck(L.hif8_transpose_bf16(gq.data_ptr(), M, N, Mp, g_t.data_ptr(), stream), "tg"),
            ck(L.hif8_transpose_bf16(xq.data_ptr(), M, K, Mp, x_t.data_ptr(), stream), "tx")),
        "wgrad_transposed_gemm": lambda: ck(L.hif8_linear_fwd_wq_split(g_t.data_ptr(), x_t.data_ptr(), None,
                                                                       gw.data_ptr(), N, K, Mp, ws.data_ptr(), ws_bytes,
                                                                       stream), "wgrad transposed"),
    }
    comparison = ("dgrad_gemm_unsplit", "wgrad_gemm_unsplit", "wgrad_transposed_transposes", "wgrad_transposed_gemm")
    for _ in range(2):
        for fn in phases.values():
            fn()
    torch.cuda.synchronize()
    times = {k: [] for k in phases}
    for _ in range(reps):
        for k, fn in phases.items():
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
            fn()
            e1.record()
            torch.cuda.synchronize()
            times[k].append(e0.elapsed_time(e1))
    ms = {k: round(sum(v) / len(v), 4) for k, v in times.items()}
    flops = 2.0 * M * N * K
    out = {"what": f"FFN-up HIF8Linear backward at x[{M},{K}], W[{N},{K}]: grad_q (224), dgrad, wgrad",
           "phases_ms": ms,
           "dgrad_TFLOPs": round(flops / (ms["dgrad_gemm"] * 1e-3) / 1e12, 1),
           "dgrad_frac": round(flops / (ms["dgrad_gemm"] * 1e-3) / 1e12 / PEAK_BF16_TFLOPS, 4),
           "wgrad_TFLOPs": round(flops / (ms["wgrad_gemm"] * 1e-3) / 1e12, 1),
           "wgrad_frac": round(flops / (ms["wgrad_gemm"] * 1e-3) / 1e12 / PEAK_BF16_TFLOPS, 4),
           "wgrad_transposed_route_TFLOPs": round(
               flops / ((ms["wgrad_transposed_gemm"] + ms["wgrad_transposed_transposes"]) * 1e-3) / 1e12, 1),
           "dgrad_unsplit_frac": round(flops / (ms["dgrad_gemm_unsplit"] * 1e-3) / 1e12 / PEAK_BF16_TFLOPS, 4),
           "wgrad_unsplit_frac": round(flops / (ms["wgrad_gemm_unsplit"] * 1e-3) / 1e12 / PEAK_BF16_TFLOPS, 4),
           "split_workspace_bytes": {"dgrad": ws_d_bytes, "wgrad": ws_bytes},
           "backward_ms": round(sum(v for k, v in ms.items() if k not in comparison), 4)}
    # hipBLASLt on the same operands (context only): grad_q @ w_q and grad_q^T @ x_q
    try:
        w_q = packed.dequantize()
        vt = {}
        for label, fn in (("dgrad", lambda: gq @ w_q), ("wgrad", lambda: gq.t() @ xq)):
            fn()
            torch.cuda.synchronize()
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
            for _ in range(reps):
                fn()
            e1.record()
            torch.cuda.synchronize()
            vt[f"{label}_ms"] = round(e0.elapsed_time(e1) / reps, 4)
        out["vendor_bf16_gemm"] = vt
        del w_q
    except Exception as ex:  # informative only
        out["vendor_bf16_gemm"] = {"error": str(ex)}
    del gy, gq, g_t, x_t, gx, gw, w_qt, xq
    torch.cuda.empty_cache()
    return out


def time_modln(pkg, torch, x, reps):
    """The modulated LayerNorm producer (osp_next.py:941 with want2v.py:96-106) in front of the
    q/k/v projections, on x: the fused two-pass route (hif8_modln_amax + hif8_modln_fake_quant)
    against the reference's sequence on the GPU (layer norm, bf16 modulation ops, then the
    _quant each of q, k and v runs on the same input)."""
    M, D = x.shape
    g = torch.Generator(device=x.device).manual_seed(4)
    e = (torch.randn(1, 6, D, generator=g, device=x.device) * 0.5).to(torch.bfloat16).chunk(6, dim=1)
    xb = x.view(1, M, D)
    L = pkg._lib.load()
    stream = pkg._lib.stream_ptr(x.device)
    stats = torch.empty(M * 2, dtype=torch.float32, device=x.device)
    st = pkg.QuantState(x.device)
    xq = torch.empty_like(x)
    sh, sc = e[0].reshape(1, D).contiguous(), e[1].reshape(1, D).contiguous()

    def p1():
        pkg._lib.check(L.hif8_modln_amax(x.data_ptr(), sh.data_ptr(), sc.data_ptr(), M, D, M, 1e-6,
                                         stats.data_ptr(), 15.0, st.ptr, stream), "hif8_modln_amax")

    def p2():
        pkg._lib.check(L.hif8_modln_fake_quant(x.data_ptr(), sh.data_ptr(), sc.data_ptr(), M, D, M,
                                               stats.data_ptr(), st.ptr, 0, xq.data_ptr(), None, stream),
                       "hif8_modln_fake_quant")

    def unfused():
        y = pkg.modulate(pkg.WanLayerNorm(D).to(x.device)(xb), e[0], e[1])
        for _ in range(3):
            pkg._quant(y, 15.0)

    def timed(fn, n):
        for _ in range(2):
            fn()
        torch.cuda.synchronize()
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        for _ in range(n):
            fn()
        b.record()
        torch.cuda.synchronize()
        return a.elapsed_time(b) / n

    with torch.no_grad():
        t1, t2 = timed(p1, reps), timed(p2, reps)
        tu = timed(unfused, max(2, reps // 4))
    n = M * D
    out = {"what": f"x_q = _quant(norm(x)*(1+scale)+shift) for q/k/v, x[{M},{D}] bf16, one modulation row",
           "amax_us": round(t1 * 1e3, 1), "qdq_us": round(t2 * 1e3, 1), "fused_us": round((t1 + t2) * 1e3, 1),
           "bytes_algorithmic": 6 * n,
           "achieved_GBps": round(6 * n / ((t1 + t2) * 1e-3) / 1e9, 1),
           "amax_GBps": round(2 * n / (t1 * 1e-3) / 1e9, 1), "qdq_GBps": round(4 * n / (t2 * 1e-3) / 1e9, 1),
           "unfused_us": round(tu * 1e3, 1), "speedup": round(tu / (t1 + t2), 2)}
    out["frac"] = round(out["achieved_GBps"] / PEAK_HBM_GBPS, 4)
    out["traffic"] = measured_traffic("k_modln_amax+k_modln_qdq")
    del stats, xq
    return out


def time_qkv(pkg, torch, x, reps):
    """The self-attention q/k/v projections (osp_next.py:742-744, 3 x [5120 -> 5120]) on the same
    x_q: one grouped launch (hif8_linear_fwd_grouped) against three single-weight launches."""
    M, K = x.shape
    g = torch.Generator(device=x.device).manual_seed(5)
    packs, biases = [], []
    for _ in range(3):
        w = (torch.randn(K, K, generator=g, device=x.device) * 0.02).to(torch.bfloat16)
        packs.append(pkg.PackedWeight(w, 15.0))
        biases.append((torch.randn(K, generator=g, device=x.device) * 0.1).to(torch.bfloat16))
        del w
    gw = pkg.GroupedWeight(packs, biases)
    a, fmt, st = pkg.quantize_activation(x, 15.0, "bf16")

    def grouped():
        return pkg.linear_fwd_grouped(a, gw)

    def separate():
        return [pkg.linear_fwd(a, fmt, st, p, b) for p, b in zip(packs, biases)]

    out = {}
    for label, fn in (("grouped", grouped), ("separate", separate)):
        for _ in range(2):
            fn()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(reps):
            fn()
        e1.record()
        torch.cuda.synchronize()
        out[f"{label}_ms"] = round(e0.elapsed_time(e1) / reps, 4)
    flops = 3 * 2.0 * M * K * K
    out["grouped_TFLOPs"] = round(flops / (out["grouped_ms"] * 1e-3) / 1e12, 1)
    out["separate_TFLOPs"] = round(flops / (out["separate_ms"] * 1e-3) / 1e12, 1)
    out["what"] = f"q, k, v [5120 -> 5120] on x_q[{M},{K}], one grouped launch vs three launches"
    del gw, packs, a
    return out


def _dit_inputs(torch, dev, g, tokens, dim, L, text_dim=None):
    x = torch.randn(1, tokens, dim, generator=g, device=dev).to(torch.bfloat16)
    e = torch.randn(1, 6, dim, generator=g, device=dev).to(torch.bfloat16)
    text = torch.randn(1, L, text_dim or dim, generator=g, device=dev).to(torch.bfloat16)
    return x, e, text


def _linear_flops(rows, dim, ffn, L):
    """FLOPs of one block's linears: self q/k/v/o and cross q/o on the block's rows, cross k/v on
    the text, FFN up/down."""
    return 2.0 * rows * dim * dim * 6 + 2.0 * L * dim * dim * 2 + 2.0 * rows * dim * ffn * 2


def time_block(pkg, torch, reps, routes=("fused", "reference"), quant_attn=None):
    """one 14B block at 720P (x [1, 75600, 5120], grid 21x45x80 padded to 48
    rows -> 4 x 20160 tokens), a Skiparse token block entered from full order, every linear HiF8
    with prepacked weights, dense bf16 attention within the 4 strided sub-grids, cross-attention
    over 512 text tokens.  Times the fused route (attention on the library's kernel) and the
    reference-order route (SDPA) (``routes``).  ``quant_attn="hif8"``: Q/K/V quantised before
    the attention, as the reference's 14B HiF8 inference config sets it."""
    D = pkg.dit
    dev = torch.device("cuda:0")
    dim, ffn, heads, grid, L = 5120, 13824, 40, (21, 45, 80), 512
    torch.manual_seed(4)
    blk = D.OSPNextAttentionBlock(dim, ffn, heads, cross_attn_norm=True, sparse_ratio=2,
                                  skiparse_block_type="token", is_full2skiparse_block=True, quant="hif8",
                                  quant_attn=quant_attn, device=dev)
    g = torch.Generator(device=dev).manual_seed(4)
    D.init_block_weights(blk, 0.02, g)
    for m in blk.modules():
        if isinstance(m, pkg.HIF8Linear):
            m.prepack()
    T, H, W = grid
    x, e, text = _dit_inputs(torch, dev, g, T * H * W, dim, L)
    rope = D.SkiparseRopeWrapper(D.rope_freqs(dim // heads).to(dev))
    tm, _ = D.skiparse_masks(1, grid, 2, dev)
    rows = int(tm.numel())

    def run(fused):
        with torch.no_grad():
            return blk(x, tm, tm, e, grid, grid, rope, text, fused=fused)

    out = {"what": "one 14B DiT block at 720P (token block from full order), all linears HiF8, "
                   "prepacked weights, bf16 attention within the 2x2 strided sub-grids (fused route: the "
                   "library's attention kernel; reference order: SDPA)",
           "tokens": T * H * W, "rows_padded": rows}
    for fused in [r == "fused" for r in routes]:
        run(fused)
        torch.cuda.synchronize()
        ea, eb = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        ea.record()
        for _ in range(reps):
            run(fused)
        eb.record()
        torch.cuda.synchronize()
        out["fused_ms" if fused else "reference_order_ms"] = round(ea.elapsed_time(eb) / reps, 3)
    lf = _linear_flops(rows, dim, ffn, L)
    n = rows // 4
    valid = [int(tm[i].sum()) for i in range(4)]
    af = sum(4.0 * n * v * dim for v in valid) + 4.0 * rows * L * dim
    out["linear_TFLOP"] = round(lf / 1e12, 3)
    out["attention_TFLOP"] = round(af / 1e12, 3)
    if "fused_ms" in out:
        out["TFLOPs_fused"] = round((lf + af) / (out["fused_ms"] * 1e-3) / 1e12, 1)
    del blk, x, e, text
    torch.cuda.empty_cache()
    return out


def time_attention(pkg, torch, reps):
    """The attention of a 14B block at 720P on the library's kernel against the reference's SDPA
    branch: self-attention over the 4 strided sub-grids of 20160 tokens with the padding keys
    masked (18900 kept), 40 heads of 128; cross-attention of the 80640 rows over 512 text tokens.
    The kernel also leaves the o projection's amax (its epilogue); the amax pass over the output
    that this replaces is timed beside it."""
    D = pkg.dit
    dev = torch.device("cuda:0")
    heads, hd, grid, L = 40, 128, (21, 45, 80), 512
    tm, _ = D.skiparse_masks(1, grid, 2, dev)
    B, N = tm.shape
    g = torch.Generator(device=dev).manual_seed(6)
    q, k, v = (torch.randn(B, N, heads, hd, generator=g, device=dev).to(torch.bfloat16) for _ in range(3))
    idx, cnt = pkg.key_list(tm)
    st = pkg.QuantState(dev)

    def timed(fn, n):
        fn()
        torch.cuda.synchronize()
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        for _ in range(n):
            fn()
        b.record()
        torch.cuda.synchronize()
        return a.elapsed_time(b) / n

    kept = [int(c) for c in cnt.tolist()]
    flops = sum(4.0 * N * c * hd * heads for c in kept)
    out = {"what": f"self-attention of the 720P block: {B} sub-grids of {N} queries over their kept keys "
                   f"({kept[0]}), {heads} heads of {hd}, bf16; cross-attention of {B * N} rows over {L} text "
                   f"tokens", "self_TFLOP": round(flops / 1e12, 3)}
    with torch.no_grad():
        o = pkg.attention_fwd(q, k, v, idx, cnt, o_state=st, o_as_f32=True)
        t_k = timed(lambda: pkg.attention_fwd(q, k, v, idx, cnt, o_state=st, o_as_f32=True), reps)
        t_s = timed(lambda: D.attention_key_masked(q, k, v, tm, out_dtype=torch.bfloat16), max(2, reps // 2))
        o2 = o.reshape(-1, heads * hd)
        t_a = timed(lambda: pkg.absmax_scale(o2, 15.0, pkg.QuantState(dev), as_f32=True), reps)
        out["self"] = {"kernel_ms": round(t_k, 3), "kernel_TFLOPs": round(flops / (t_k * 1e-3) / 1e12, 1),
                       "frac_of_peak": round(flops / (t_k * 1e-3) / 1e12 / PEAK_BF16_TFLOPS, 4),
                       "sdpa_ms": round(t_s, 3), "sdpa_TFLOPs": round(flops / (t_s * 1e-3) / 1e12, 1),
                       "amax_pass_replaced_us": round(t_a * 1e3, 1)}
        del q, k, v, o, o2
        qc = torch.randn(1, B * N, heads, hd, generator=g, device=dev).to(torch.bfloat16)
        kc, vc = (torch.randn(1, L, heads, hd, generator=g, device=dev).to(torch.bfloat16) for _ in range(2))
        cflops = 4.0 * B * N * L * hd * heads
        t_kc = timed(lambda: pkg.attention_fwd(qc, kc, vc, o_state=st), reps)
        t_sc = timed(lambda: D.attention_key_masked(qc, kc, vc, None), reps)
        out["cross"] = {"kernel_ms": round(t_kc, 3), "kernel_TFLOPs": round(cflops / (t_kc * 1e-3) / 1e12, 1),
                        "sdpa_ms": round(t_sc, 3), "sdpa_TFLOPs": round(cflops / (t_sc * 1e-3) / 1e12, 1)}
    torch.cuda.empty_cache()
    return out


def time_step(pkg, torch, reps):
    """the 40-block loop of a 14B OSP-Next denoising step at 768P native
    (grid 21x48x84 = 84672 tokens, no padding), dual-end schedule with 8 full blocks, every
    block linear HiF8 with prepacked weights, text 512 x 4096 through the (bf16) text embedding.
    The patch/time embeddings and the head are not included (under 0.1 % of the FLOPs)."""
    D = pkg.dit
    dev = torch.device("cuda:0")
    dim, ffn, heads, grid, L, text_dim = 5120, 13824, 40, (21, 48, 84), 512, 4096
    torch.manual_seed(5)
    stack = D.OSPNextBlocks(dim, ffn, heads, num_layers=40, num_full_blocks=8, quant="hif8", device=dev)
    g = torch.Generator(device=dev).manual_seed(5)
    D.init_block_weights(stack, 0.02, g)
    for m in stack.modules():
        if isinstance(m, pkg.HIF8Linear):
            m.prepack(drop_weight=True)
    torch.cuda.empty_cache()
    text_embedding = torch.nn.Sequential(torch.nn.Linear(text_dim, dim), torch.nn.GELU(approximate="tanh"),
                                         torch.nn.Linear(dim, dim)).to(dev, torch.bfloat16)
    D.init_block_weights(text_embedding, 0.02, g)
    T, H, W = grid
    x, e, text_in = _dit_inputs(torch, dev, g, T * H * W, dim, L, text_dim)

    def run():
        with torch.no_grad():
            return stack(x, e, text_embedding(text_in), grid)

    run()
    torch.cuda.synchronize()
    ea, eb = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    ea.record()
    for _ in range(reps):
        run()
    eb.record()
    torch.cuda.synchronize()
    ms = ea.elapsed_time(eb) / reps
    rows = T * H * W
    lf = 40 * _linear_flops(rows, dim, ffn, L)
    out = {"what": "40-block loop of one 14B denoising step at 768P (dual-end, 8 full blocks), all block "
                   "linears HiF8, prepacked weights", "tokens": rows, "ms_per_step": round(ms, 1),
           "linear_TFLOP": round(lf / 1e12, 1), "linear_TFLOPs_over_step": round(lf / (ms * 1e-3) / 1e12, 1)}
    del stack, x, e, text_in
    torch.cuda.empty_cache()
    return out


def time_data_dependence(pkg, torch, x, w, reps):
    """The fused GEMM on the FFN-up shape with constant instead of random operands (x, W, both):
    a kernel at the board's power limit runs faster when its operands do not toggle.  Not the
    benchmark workload; reported beside it."""
    dev = x.device
    M, K = x.shape
    N = w.shape[0]
    L = pkg._lib.load()
    stream = pkg._lib.stream_ptr(dev)
    y = torch.empty(M, N, dtype=torch.bfloat16, device=dev)

    def operands(xx, ww):
        st = pkg.absmax_scale(xx, 15.0, pkg.QuantState(dev))
        return pkg.fake_quant(xx, st), pkg.PackedWeight(ww, 15.0)

    def gemm_ms(xq, pw):
        def run():
            pkg._lib.check(L.hif8_linear_fwd(xq.data_ptr(), pw.codes.data_ptr(), pw.state.ptr, None, y.data_ptr(),
                                             M, N, K, stream), "linear")
        run()
        torch.cuda.synchronize()
        ea, eb = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        ea.record()
        for _ in range(reps):
            run()
        eb.record()
        torch.cuda.synchronize()
        return round(ea.elapsed_time(eb) / reps, 3)

    xc = torch.full_like(x, 0.5)
    wc = torch.full_like(w, 0.01)
    out = {"what": "k_linear_dtl ms at the FFN-up shape by operand data (x / W)"}
    xr_q, wr_p = operands(x, w)
    xc_q, wc_p = operands(xc, wc)
    out["random/random"] = gemm_ms(xr_q, wr_p)
    out["random/const"] = gemm_ms(xr_q, wc_p)
    out["const/random"] = gemm_ms(xc_q, wr_p)
    out["const/const"] = gemm_ms(xc_q, wc_p)
    del xc, wc, xr_q, wr_p, xc_q, wc_p, y
    return out


def median(v):
    s = sorted(v)
    return s[len(s) // 2]


def _cpu_info():
    """The host CPU as ``lscpu`` names it, the identifying fields it prints beside the model name
    (which a virtual machine may shorten, e.g. to "AMD EPYC"), and the instruction-set flags that
    decide its bf16 GEMM rate (AMX, AVX-512 BF16): ``(model, details, {flag: present})``.
    /proc/cpuinfo when lscpu is absent."""
    model, flags, details = None, set(), {}
    keep = {"Vendor ID": "vendor", "CPU family": "family", "Model": "model_number", "Stepping": "stepping",
            "Hypervisor vendor": "hypervisor", "Socket(s)": "sockets", "Core(s) per socket": "cores_per_socket",
            "Thread(s) per core": "threads_per_core", "L3": "l3"}
    try:
        import subprocess
        out = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=20).stdout
        for line in out.splitlines():
            key, _, val = line.partition(":")
            key = key.strip()
            if key == "Model name" and model is None:
                model = val.strip()
            elif key == "Flags":
                flags = set(val.split())
            elif key in keep and keep[key] not in details:
                details[keep[key]] = val.strip()
    except Exception:
        pass
    if model is None or not flags:
        try:
            with open("/proc/cpuinfo") as f:
                for line in f:
                    key, _, val = line.partition(":")
                    if key.strip() == "model name" and model is None:
                        model = val.strip()
                    elif key.strip() == "flags" and not flags:
                        flags = set(val.split())
        except OSError:
            pass
    names = ("amx_bf16", "amx_tile", "amx_int8", "avx512_bf16", "avx512f", "avx512_vnni", "avx2")
    return model or platform.machine(), details, {n: n in flags for n in names}


def _mem_available():
    """MemAvailable from /proc/meminfo in bytes (None where it cannot be read)."""
    try:
        with open("/proc/meminfo") as f:
            for line in f:
                if line.startswith("MemAvailable:"):
                    return int(line.split()[1]) * 1024
    except (OSError, ValueError, IndexError):
        pass
    return None


def _cpu_threads():
    """Threads for the CPU baseline: every CPU this process may run on (its affinity set), capped
    by OMP_NUM_THREADS when the environment sets it (the GPU box grants each one-GPU job a CPU
    share and sets OMP_NUM_THREADS to it)."""
    try:
        n = len(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        n = os.cpu_count() or 1
    omp = os.environ.get("OMP_NUM_THREADS", "")
    if omp.isdigit() and int(omp) > 0:
        n = min(n, int(omp))
    return max(1, n)


def _time_cpu(fn, warm, max_runs=3, budget_s=15.0):
    """One warm-up call of ``warm``, then the median of up to ``max_runs`` calls of ``fn`` (fewer when
    a call takes more than ``budget_s``); returns (median seconds, runs)."""
    warm()
    ts = []
    for _ in range(max_runs):
        t0 = time.perf_counter()
        fn()
        ts.append(time.perf_counter() - t0)
        if ts[-1] > budget_s:
            break
    return median(ts), len(ts)


def cpu_baseline(torch, M, K, N, sample_rows=4096, target_s=10.0):
    """The reference CPU path (torch ops: _quant + quant_hif8 + F.linear in bf16) on the host.

    Headline (``value``): the 14B FFN-up step.  A [sample_rows, K] slice of x (quantise + GEMM
    against the quantised W) is repeated until about ``target_s`` seconds of CPU work, and the
    per-call weight quantisation runs twice; the step estimate is the weight part plus the slice
    time scaled to M (both the qdq and the GEMM are linear in M).  When the host has the memory
    (twice the ~12 GB the step holds), the whole step then runs once at M rows and ``value`` is
    that run; otherwise ``value`` is the estimate.  Beside it, BASELINE config 1 (the qdq of a
    [4096, 5120] tensor) and config 2 (the three Wan-1.3B 480P linears) at full size: a warm-up
    on a slice, then the median of three runs."""
    sys.path.insert(0, ROOT)
    import numpy as np
    import torch.nn.functional as F
    from oracle import hif8_ref as R

    threads = _cpu_threads()
    torch.set_num_threads(threads)
    g = torch.Generator().manual_seed(0)
    x = torch.randn(sample_rows, K, generator=g)
    x[:, torch.randperm(K, generator=g)[:16]] *= 20
    x = x.to(torch.bfloat16)
    w = (torch.randn(N, K, generator=g) * 0.02).to(torch.bfloat16)
    R.quant_torch_cpu(x[:64], 15.0)  # warm
    t_start = time.perf_counter()
    t_w = []
    for _ in range(2):
        t0 = time.perf_counter()
        wq, _ = R.quant_torch_cpu(w, 15.0)
        t_w.append(time.perf_counter() - t0)
    F.linear(x[:64], wq)  # warm
    t_slice = []
    while True:
        t0 = time.perf_counter()
        xq, _ = R.quant_torch_cpu(x, 15.0)
        F.linear(xq, wq)
        t_slice.append(time.perf_counter() - t0)
        if time.perf_counter() - t_start >= target_s or len(t_slice) >= 200:
            break
    total = time.perf_counter() - t_start
    tw, ts = median(t_w), median(t_slice)
    t_est = tw + (M / sample_rows) * ts
    del xq

    # the whole step at M rows, once, when the host has room for it (x, its fp32 temporaries
    # and the [M, N] bf16 output: about 12 GB at the 14B FFN-up shape); x is the slice tiled to M
    # rows, so its amax is the slice's
    full = None
    need = 4 * M * K * 4 + 2 * M * N
    avail = _mem_available()
    if avail is not None and avail >= 2 * need:
        reps = -(-M // sample_rows)
        xf = x.repeat(reps, 1)[:M].contiguous()
        t0 = time.perf_counter()
        wq2, _ = R.quant_torch_cpu(w, 15.0)
        xq, _ = R.quant_torch_cpu(xf, 15.0)
        y = F.linear(xq, wq2)
        t_one = time.perf_counter() - t0
        full = {"M": M, "s": round(t_one, 3), "TFLOPs": round(2.0 * M * N * K / t_one / 1e12, 4),
                "what": "W qdq + x qdq + bf16 F.linear at full size, one run (its first touch of "
                        "the output and temporaries included, as in the reference's own call)"}
        del xf, xq, y, wq2
    t_full = full["s"] if full else t_est
    value = 2.0 * M * N * K / t_full / 1e12
    del x, w, wq

    # config 1: _quant of the [4096, 5120] bf16 tensor (N(0, 0.02), 0.1 % outliers x50, seed 0)
    c1_bits = R.c1_input(0)
    c1 = torch.from_numpy(c1_bits.view(np.int16)).view(torch.bfloat16)
    t_c1, n_c1 = _time_cpu(lambda: R.quant_torch_cpu(c1, 15.0), lambda: R.quant_torch_cpu(c1[:256], 15.0))
    c1_out = {"what": "_quant (torch-path qdq) of x[4096,5120] bf16", "s": round(t_c1, 4), "runs": n_c1,
              "GBps_algorithmic": round(4.0 * c1.numel() / t_c1 / 1e9, 3)}
    del c1
    # config 2: Wan-1.3B 480P, x [32760, 1536] N(0,1) with 8 outlier channels x20 (seed 1); the FFN-down
    # input is [32760, 8960] from the same recipe; W N(0, 0.02) (seeds 2, 3, 4), zero bias
    c2 = {}
    Mc = 32760
    for name, n_, k_, seed in (("qkvo", 1536, 1536, 2), ("ffn_up", 8960, 1536, 3), ("ffn_down", 1536, 8960, 4)):
        gx = torch.Generator().manual_seed(1)
        xc = torch.randn(Mc, k_, generator=gx)
        xc[:, torch.randperm(k_, generator=gx)[:8]] *= 20
        xc = xc.to(torch.bfloat16)
        wc = (torch.randn(n_, k_, generator=torch.Generator().manual_seed(seed)) * 0.02).to(torch.bfloat16)
        bc = torch.zeros(n_, dtype=torch.bfloat16)
        t_c, n_c = _time_cpu(lambda: R.linear_torch_cpu(xc, wc, bc), lambda: R.linear_torch_cpu(xc[:512], wc, bc))
        c2[name] = {"M": Mc, "N": n_, "K": k_, "s": round(t_c, 4), "runs": n_c,
                    "TFLOPs": round(2.0 * Mc * n_ * k_ / t_c / 1e12, 4)}
        del xc, wc, bc
    model, details, flags = _cpu_info()
    return {
        "value": round(value, 4), "unit": "TFLOP/s", "cores": threads, "kind": "port",
        "sample": ((f"one full step at M={M} ({t_full:.2f}s); " if full else
                    f"no full-size step (host memory available {avail} B, wanted {2 * need} B); ") +
                   f"reference CPU path (torch ops, bf16 F.linear) on the FFN-up shape: W[{N},{K}] qdq x2 "
                   f"(median {tw:.2f}s) and {len(t_slice)} reps of an x[{sample_rows},{K}] slice, qdq + GEMM "
                   f"(median {ts:.3f}s), {total:.1f}s of CPU work; estimated step at M={M} = W qdq + "
                   f"{M / sample_rows:.2f} slices = {t_est:.2f}s"),
        "full_step": full, "slice_estimate_s": round(t_est, 3),
        "cpu_model": model, "cpu_lscpu": details, "cpu_flags": flags, "os_cpu_count": os.cpu_count(),
        "affinity_cpus": len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else None,
        "omp_num_threads": os.environ.get("OMP_NUM_THREADS"),
        "c1": c1_out, "c2": c2,
    }


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--route", default="auto", choices=["auto", "fused", "decode_once"],
                    help="GEMM route for bf16 activations (auto: HIF8Linear's rule, decode_once at this M)")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--shapes", default="up,bwd,ffn,down,qkvo,c2,modln,qkv,attn,block,block_qa,step",
                    help="comma list of up,bwd (the FFN-up backward),down,qkvo (the other 14B linears),"
                         "c2 (the three 1.3B 480P linears, config 2),ffn,modln,qkv,attn (the block's "
                         "attention with the o amax epilogue),block (config 4),block_qa (config 4 with "
                         "quant_attn=hif8),step (config 5),"
                         "data (the GEMM with constant operands) to time in addition")
    ap.add_argument("--block-routes", default="fused,reference",
                    help="routes of the block (config 4) to time: fused, reference or both")
    ap.add_argument("--pmc-calibration", action="store_true",
                    help="also run one plain copy of x (774,144,000 B read + written): the reference "
                         "kernel for scaling rocprofv3 FETCH_SIZE / WRITE_SIZE")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py: this build targets one GPU (no collectives); run with --gpus 1", file=sys.stderr)
        sys.exit(2)

    import torch
    sys.path.insert(0, ROOT)
    from __graft_entry__ import load_package
    pkg = load_package()
    pkg._lib.load()
    dev = torch.device("cuda:0")
    M, K, N = 75600, 5120, 13824

    log(f"[bench] inputs M={M} K={K} N={N}")
    x, w, b = make_inputs(torch, M, K, N)
    packed = pkg.PackedWeight(w, 15.0)
    if args.pmc_calibration:
        xc = torch.empty_like(x)
        xc.copy_(x)
        torch.cuda.synchronize()
        del xc
    torch.cuda.synchronize()
    route = args.route
    if route == "auto":   # HIF8Linear's own choice for bf16 activations (hif8_linear.decode_once)
        route = "decode_once" if pkg.hif8_linear.decode_once(M, K) else "fused"
    log(f"[bench] timing FFN-up step ({route})")
    r = time_linear(pkg, torch, x, packed, b, args.steps, args.warmup, route)
    step_ms = [a + q + d + g for a, q, d, g in zip(r["amax"], r["quant"], r["wdecode"], r["gemm"])]
    ms_step = r["wall_ms"] / args.steps
    flops = 2.0 * M * N * K
    value = flops / (ms_step * 1e-3) / 1e12
    gemm_ms = sum(r["gemm"]) / len(r["gemm"])
    amax_ms = sum(r["amax"]) / len(r["amax"])
    quant_ms = sum(r["quant"]) / len(r["quant"])
    wdec_ms = sum(r["wdecode"]) / len(r["wdecode"])
    gemm_tflops = flops / (gemm_ms * 1e-3) / 1e12
    # the other route on the same operands, for comparison
    other = "fused" if route == "decode_once" else "decode_once"
    other_route = None
    if other:
        ro = time_linear(pkg, torch, x, packed, b, max(3, args.steps // 2), 1, other)
        og = sum(ro["gemm"]) / len(ro["gemm"])
        od = sum(ro["wdecode"]) / len(ro["wdecode"])
        other_route = {"route": other, "gemm_ms": round(og, 4), "wdecode_ms": round(od, 4),
                       "gemm_TFLOPs": round(flops / (og * 1e-3) / 1e12, 1),
                       "kernel": "k_linear_w16" if other == "decode_once" else "k_linear_dtl"}
        del ro
    n = M * K
    enc_bytes = 6 * n   # amax read + fake-quant read/write
    enc_gbps = enc_bytes / ((amax_ms + quant_ms) * 1e-3) / 1e9

    # encode (codes) throughput, the bandwidth headline: amax + encode of x
    st = pkg.QuantState(dev)
    codes = torch.empty((M, K), dtype=torch.uint8, device=dev)
    L = pkg._lib.load()
    stream = pkg._lib.stream_ptr(dev)
    for _ in range(2):
        L.hif8_absmax_scale(x.data_ptr(), 0, n, 15.0, st.ptr, stream)
        L.hif8_encode(x.data_ptr(), 0, n, st.ptr, codes.data_ptr(), stream)
    torch.cuda.synchronize()
    e0, e1, e2 = (torch.cuda.Event(enable_timing=True) for _ in range(3))
    ta, te = [], []
    for _ in range(args.steps):
        e0.record()
        pkg._lib.check(L.hif8_absmax_scale(x.data_ptr(), 0, n, 15.0, st.ptr, stream), "amax")
        e1.record()
        pkg._lib.check(L.hif8_encode(x.data_ptr(), 0, n, st.ptr, codes.data_ptr(), stream), "encode")
        e2.record()
        torch.cuda.synchronize()
        ta.append(e0.elapsed_time(e1))
        te.append(e1.elapsed_time(e2))
    enc_ms = sum(ta) / len(ta) + sum(te) / len(te)
    encode = {
        "workload": f"amax+scale+encode of x[{M},{K}] bf16 -> uint8 codes",
        "bytes_algorithmic": 5 * n, "ms": round(enc_ms, 4),
        "achieved_GBps": round(5 * n / (enc_ms * 1e-3) / 1e9, 1),
        "amax_ms": round(sum(ta) / len(ta), 4), "encode_ms": round(sum(te) / len(te), 4),
        "amax_GBps": round(2 * n / (sum(ta) / len(ta) * 1e-3) / 1e9, 1),
        "encode_kernel_GBps": round(3 * n / (sum(te) / len(te) * 1e-3) / 1e9, 1),
        "peak_GBps": PEAK_HBM_GBPS,
    }
    encode["frac"] = round(encode["achieved_GBps"] / PEAK_HBM_GBPS, 4)
    encode["traffic"] = measured_traffic("k_absmax+k_quant_encode")
    # streaming references with torch's own elementwise kernels on the same x (context only):
    # a copy (2 B read + 2 B written per element) and a cast to uint8 (2 B read + 1 B written,
    # the encode kernel's traffic shape)
    refs = {}
    for name, dst, nbytes in (("copy", torch.empty_like(x), 4 * n), ("cast_u8", codes, 3 * n)):
        dst.copy_(x)
        torch.cuda.synchronize()
        ea, eb = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        ea.record()
        for _ in range(5):
            dst.copy_(x)
        eb.record()
        torch.cuda.synchronize()
        refs[name + "_GBps"] = round(nbytes / (ea.elapsed_time(eb) / 5 * 1e-3) / 1e9, 1)
    encode["torch_streaming_refs"] = refs
    del codes

    extra_shapes = {}
    if "ffn" in args.shapes.split(","):
        log("[bench] timing the FFN (GELU route)")
        try:
            extra_shapes["ffn"] = time_ffn(pkg, torch, x, max(3, args.steps // 2))
        except Exception as ex:
            extra_shapes["ffn"] = {"error": repr(ex)}
    if "bwd" in args.shapes.split(","):
        log("[bench] timing the FFN-up backward (dgrad, wgrad)")
        try:
            extra_shapes["bwd"] = time_backward(pkg, torch, x, packed, max(3, args.steps // 4))
        except Exception as ex:
            extra_shapes["bwd"] = {"error": repr(ex)}
    if "modln" in args.shapes.split(","):
        log("[bench] timing the modulated LayerNorm producer")
        extra_shapes["modln"] = time_modln(pkg, torch, x, max(5, args.steps))
    if "qkv" in args.shapes.split(","):
        log("[bench] timing the grouped q/k/v projections")
        extra_shapes["qkv"] = time_qkv(pkg, torch, x, max(3, args.steps // 4))
    if "data" in args.shapes.split(","):
        log("[bench] timing the fused GEMM with constant operands")
        extra_shapes["data"] = time_data_dependence(pkg, torch, x, w, max(3, args.steps // 2))
    if "attn" in args.shapes.split(","):
        log("[bench] timing the block's attention (kernel with the o amax epilogue, and SDPA)")
        try:
            extra_shapes["attn"] = time_attention(pkg, torch, max(3, args.steps // 4))
        except Exception as ex:
            extra_shapes["attn"] = {"error": repr(ex)}
    if "block" in args.shapes.split(","):
        log("[bench] timing one 14B DiT block at 720P (config 4)")
        try:
            extra_shapes["block"] = time_block(pkg, torch, 3, tuple(args.block_routes.split(",")))
        except Exception as ex:  # the harness around the path (attention backend) may be missing
            extra_shapes["block"] = {"error": repr(ex)}
    if "block_qa" in args.shapes.split(","):
        log("[bench] timing one 14B DiT block at 720P with quant_attn=hif8")
        try:
            extra_shapes["block_qa"] = time_block(pkg, torch, 3, ("fused",), quant_attn="hif8")
        except Exception as ex:
            extra_shapes["block_qa"] = {"error": repr(ex)}
    if "step" in args.shapes.split(","):
        log("[bench] timing the 40-block denoising step at 768P (config 5)")
        try:
            extra_shapes["step"] = time_step(pkg, torch, 2)
        except Exception as ex:
            extra_shapes["step"] = {"error": repr(ex)}
    def linear_line(m_, n_, k_, seed, outliers):
        xs, ws, bs = make_inputs(torch, m_, k_, n_, seed=seed, outlier_channels=outliers)
        ps = pkg.PackedWeight(ws, 15.0)
        r_ = route if args.route != "auto" else ("decode_once" if pkg.hif8_linear.decode_once(m_, k_) else "fused")
        rr = time_linear(pkg, torch, xs, ps, bs, max(3, args.steps // 2), 2, r_)
        gm = sum(rr["gemm"]) / len(rr["gemm"])
        st_ms = rr["wall_ms"] / max(3, args.steps // 2)
        line = {"M": m_, "N": n_, "K": k_, "route": r_, "gemm_ms": round(gm, 4),
                "gemm_TFLOPs": round(2.0 * m_ * n_ * k_ / (gm * 1e-3) / 1e12, 1),
                "gemm_frac": round(2.0 * m_ * n_ * k_ / (gm * 1e-3) / 1e12 / PEAK_BF16_TFLOPS, 4),
                "step_ms": round(st_ms, 4),
                "step_TFLOPs": round(2.0 * m_ * n_ * k_ / (st_ms * 1e-3) / 1e12, 1)}
        del xs, ws, bs, ps, rr
        return line

    for name in [s for s in args.shapes.split(",")
                 if s and s not in ("up", "bwd", "ffn", "modln", "qkv", "attn", "block", "block_qa", "step", "data",
                                    "c2")]:
        n_, k_ = {"down": (5120, 13824), "qkvo": (5120, 5120)}[name]
        print(f"[bench] timing the 14B {name} linear", file=sys.stderr, flush=True)
        extra_shapes[name] = linear_line(M, n_, k_, 1, 16)
    if "c2" in args.shapes.split(","):
        # config 2: the 1.3B 480P linears on x [32760, 1536] with 8 outlier channels
        print("[bench] timing the 1.3B 480P linears (config 2)", file=sys.stderr, flush=True)
        extra_shapes["c2"] = {name: linear_line(32760, n_, k_, seed, 8)
                              for name, n_, k_, seed in (("qkvo", 1536, 1536, 2), ("ffn_up", 8960, 1536, 3),
                                                         ("ffn_down", 1536, 8960, 4))}
        try:
            extra_shapes["c2"]["module_eager_vs_graph"] = time_module_graph(pkg, torch, 32760, args.steps)
        except Exception as ex:  # informative only
            extra_shapes["c2"]["module_eager_vs_graph"] = {"error": repr(ex)}

    # the vendor bf16 GEMM on the same shape, for context (not part of the product)
    vendor = None
    try:
        xq = pkg.fake_quant(x, pkg.absmax_scale(x, 15.0, pkg.QuantState(dev)))
        wq = packed.dequantize()
        for _ in range(2):
            torch.nn.functional.linear(xq, wq, b)
        torch.cuda.synchronize()
        ea, eb = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        ea.record()
        for _ in range(5):
            torch.nn.functional.linear(xq, wq, b)
        eb.record()
        torch.cuda.synchronize()
        vms = ea.elapsed_time(eb) / 5
        vendor = {"what": "torch F.linear (hipBLASLt) bf16 on the dequantised operands", "ms": round(vms, 4),
                  "TFLOPs": round(flops / (vms * 1e-3) / 1e12, 1)}
        del xq, wq
    except Exception as ex:  # informative only
        vendor = {"error": str(ex)}

    cpu = None
    if not args.no_cpu:
        log("[bench] CPU baseline")
        try:
            cpu = cpu_baseline(torch, M, K, N)
        except Exception as ex:
            cpu = {"error": str(ex)}

    kernel_name = "k_linear_dtl"
    if route == "decode_once":
        kernel_name = "k_linear_w16"
    gemm_desc = ("weight codes decoded once to bf16 (hif8_decode) -> decode-free HiF8 GEMM (k_linear_w16)"
                 if route == "decode_once" else "fused HiF8 dequant-GEMM")
    out = {
        "metric": METRIC,
        "value": round(value, 2),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {
            "workload": ("Wan-14B 720P FFN-up HIF8Linear forward: x[75600,5120] bf16 -> amax+scale -> "
                         f"fake-quant (bf16) -> {gemm_desc} "
                         "(W[13824,5120] held as packed 8-bit HiF8, bias) -> y bf16"),
            "M": M, "K": K, "N": N, "route": route, "scale_max": 15.0,
        },
        "roofline": {
            "kernel": kernel_name,
            "bound": "mfma",
            "achieved": round(gemm_tflops, 2),
            "peak": PEAK_BF16_TFLOPS,
            "unit": "TFLOP/s",
            "frac": round(gemm_tflops / PEAK_BF16_TFLOPS, 4),
            "traffic": measured_traffic(kernel_name),
            "traffic_source": "profiles/hif8_kernels_14b_720p_hbm_traffic.md (rocprofv3 FETCH_SIZE x2 + WRITE_SIZE)",
            "gemm_ms": round(gemm_ms, 4),
        },
        "phases_ms": {"amax": round(amax_ms, 4), "quant": round(quant_ms, 4), "weight_decode": round(wdec_ms, 4),
                      "gemm": round(gemm_ms, 4), "events_sum": round(median(step_ms), 4)},
        "other_route": other_route,
        "act_quant_GBps": round(enc_gbps, 1),
        "encode": encode,
        "shapes": extra_shapes,
        "vendor_bf16_gemm": vendor,
        "cpu_baseline": cpu,
    }
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
