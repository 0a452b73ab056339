#!/usr/bin/env python3
"""Benchmark: CosyVoice3 Flow DiT Euler-step mel frames/s at T=500, B=2 (CFG pair).

One "step" is one device-resident CFG Euler step of the full 22-block DiT
estimator (time MLP + stacked AdaLN GEMV + input embedding + 22 blocks +
norm_out/proj_out + CFG combine/x update), inputs resident in HBM.
value = T * steps / wall time of the timed region (mel frames per second).

Also reported on the same JSON line:
  roofline      the dominant kernel's achieved fp32 FLOP/s (HIP events around graph
                replays of its launches under continuous load, on the replay stream)
                vs the 157.3 TFLOP/s fp32 matrix peak (for a split-operand kernel,
                which forms each fp32 product from three bf16 MFMA products (the
                estimator's default; six in its fp32-GEMM-level mode), also
                the bf16 MFMA flops executed vs the 2.5 PFLOP/s dense bf16 peak, as
                bf16_pipe), and its HBM traffic per launch from the committed
                rocprofv3 FETCH_SIZE / WRITE_SIZE summary;
  six_products  the same timed steps with the block projections and attention on
                the six-product split (fp32-GEMM error level;
                lx_dit_set_products(dit, 6));
  kernels       per-kernel-class timings of one step's launches (same method), each
                class on the kernel the estimator runs for it;
  fused_ops     achieved HBM GB/s of every fused op at the configs' shapes, with
                each launch on a distinct buffer set (> 256 MB rotation, so the
                MALL does not serve the reads);
  stream_ceiling the library's own streaming rate (its GELU over 1 GiB moved);
  flow_infer    the whole FlowDecoder inference of a 10 s utterance (frontend +
                10 Euler steps), host token ids in, output mel frames out;
  cpu_baseline  the reference's fp32 ggml graph for the same Euler step, restated
                node by node on this host's cores (bounded sample).

Usage: python bench.py [--steps K] [--warmup W] [--T 500] [--no-cpu]
"""
import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
MFMA_F32_PEAK_TFLOPS = 157.3
MFMA_BF16_PEAK_TFLOPS = 2500.0
# bf16 MFMA products per fp32 product in the estimator's split-operand
# projections and attention (its default, lx_dit.cpp `products`)
DIT_PRODUCTS = 3


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--T", type=int, default=500)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--cpu-seconds", type=float, default=12.0)
    ap.add_argument("--no-fused", action="store_true", help="skip the fused-op GB/s sweep")
    ap.add_argument("--no-llm", action="store_true", help="skip the Qwen2 prefill/decode timing")
    ap.add_argument("--no-flow", action="store_true",
                    help="skip the whole-utterance FlowDecoder inference timing")
    ap.add_argument("--counter-probe", action="store_true",
                    help="only launch the T=500 QKV and FF0 projections and attention, for "
                         "rocprofv3 --pmc passes (matrix-core, VALU and LDS counters)")
    ap.add_argument("--traffic-probe", action="store_true",
                    help="only launch the dominant GEMM (QKV + rotary, T=500) and a plain "
                         "device copy of known size, for rocprofv3 --pmc FETCH_SIZE/WRITE_SIZE")
    ap.add_argument("--prefill-probe", action="store_true",
                    help="only run the Qwen2 prefill (L=256, 24 layers) ten times, for "
                         "rocprofv3 --pmc passes over its kernels")
    return ap.parse_args()


def profiled_kernels(torch, fn):
    """Kernel launches of fn() as the HIP runtime records them (torch.profiler's
    device activity: every launch on the device, including liblxops's own):
    [(name, start_us, duration_us)] in launch order."""
    from torch.profiler import ProfilerActivity, profile
    torch.cuda.synchronize()
    with profile(activities=[ProfilerActivity.CUDA]) as prof:
        fn()
        torch.cuda.synchronize()
    out = []
    for e in prof.events():
        if str(getattr(e, "device_type", "")).endswith("CUDA"):
            dur = e.device_time if hasattr(e, "device_time") else e.cuda_time
            out.append((e.name, e.time_range.start, dur))
    out.sort(key=lambda r: r[1])
    return out


def kernel_gbs(records, match, nbytes, note):
    """Average duration of the launches whose name contains `match` and their
    algorithmic GB/s; nbytes is one number or a per-launch list (cycled)."""
    durs = [d for n, _, d in records if match in n]
    if not durs:
        return None
    per = nbytes if isinstance(nbytes, (list, tuple)) else [nbytes]
    tot_b = sum(per[i % len(per)] for i in range(len(durs)))
    avg_us = sum(durs) / len(durs)
    gbs = tot_b / (sum(durs) * 1e-6) / 1e9
    return {"launches": len(durs), "avg_us": round(avg_us, 3),
            "bytes_per_launch": round(tot_b / len(durs)), "gbs": round(gbs, 1),
            "frac": round(gbs / HBM_PEAK_GBS, 4), "note": note}


def splitk_slices(M, N, K, target_wgs=512, max_slices=8):
    """K slices the library's split-K plan gives an (M, N, K) projection
    (gemm_splitk_plan in larynx_amd/csrc/lx_gemm.hip): about two workgroups per
    CU, at least four 32-wide slabs per slice, whole slab pairs."""
    tiles = ((M + 63) // 64) * ((N + 63) // 64)
    s = (target_wgs + tiles - 1) // tiles
    s = max(1, min(s, max(1, min(max_slices, K // 128))))
    ks = (K + s - 1) // s
    ks = (ks + 63) // 64 * 64
    return (K + ks - 1) // ks


def in_step_matrix(records, ops):
    """Average in-step duration of the T=500 step's matrix kernels (64-row tiles,
    the estimator's product count; with three products the activations arrive
    as two-part packed rows and FF0 writes its output packed) from activity
    records of whole steps; the out and FF2 projections share one kernel (the
    partial-product output)."""
    ap = ", 1" if DIT_PRODUCTS == 3 else ""
    ff0_out = ops.LX_BX_OUT_PACKED if DIT_PRODUCTS == 3 else ops.LX_BX_OUT_F32
    pats = {
        "gemm_qkv_rope": f"gemm_bx_kernel<{ops.LX_EPI_ROPE_PARTIAL}, 2, {ff0_out}, {DIT_PRODUCTS}{ap}>",
        "gemm_ff0_gelu": f"gemm_bx_kernel<{ops.LX_EPI_GELU_TANH}, 2, {ff0_out}, {DIT_PRODUCTS}{ap}>",
        "gemm_out_ff2_partial": f"gemm_bx_kernel<{ops.LX_EPI_NONE}, 2, 1, {DIT_PRODUCTS}{ap}>",
        "attention": f"attn_bx_kernel<2, 2, true, {DIT_PRODUCTS}"
                     + (", true>" if DIT_PRODUCTS == 3 else ">"),
    }
    out = {}
    for k, pat in pats.items():
        durs = [d for n, _, d in records if pat in n]
        out[k] = ({"launches": len(durs), "avg_us": sum(durs) / len(durs)} if durs else None)
    return out


def prefill_bx_slices(rows, N, K):
    """K slices of a Qwen2 prefill projection on the fragment-order GEMM
    (prefill_bx_slices in larynx_amd/csrc/lx_qwen2.cpp): at most 9 and at most
    256 / (64-row tiles), then the fewest with the same longest slice."""
    steps = K // 64
    tiles = ((rows + 63) // 64) * (N // 128)
    most = min(9, steps, max(1, 256 // tiles))
    per = -(-steps // most)
    return -(-steps // per)


def pack2(torch, x):
    """Two-part packed rows of an fp32 (M, K) tensor, built with torch: each
    aligned group of four values as the four bf16(x) then the four
    bf16(x - bf16(x)) (round to nearest even), in the group's 16 bytes -- the
    operand linear_bx reads with a_packed."""
    M, K = x.shape
    x0 = x.to(torch.bfloat16)
    x1 = (x - x0.float()).to(torch.bfloat16)
    both = torch.stack([x0.view(M, K // 4, 4), x1.view(M, K // 4, 4)], dim=2)
    return both.reshape(M, 2 * K).view(torch.float32).contiguous()


def event_time_ms(fn, n, torch):
    """Average ms per call of fn over n calls, HIP events on torch's current
    stream (the stream every liblxops call of this script is enqueued on)."""
    s = torch.cuda.current_stream()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    fn()
    torch.cuda.synchronize()
    a.record(s)
    for _ in range(n):
        fn()
    b.record(s)
    b.synchronize()
    return a.elapsed_time(b) / n


def steady_launch_ms(fn, torch, n=20, warm_ms=40.0, reps=10):
    """Average ms of one call of fn under continuous load: n calls captured
    into one HIP graph, replayed back to back for about warm_ms (the device's
    clocks settle under load, as they do inside a run of Euler steps), then
    `reps` more replays bracketed by a pair of HIP events on the replay stream.
    The figure includes the device-side dispatch gap between consecutive graph
    kernels (about 1 us)."""
    s = torch.cuda.Stream()
    with torch.cuda.stream(s):
        fn()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        for _ in range(n):
            fn()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    with torch.cuda.stream(s):
        a.record(s)
        g.replay()
        b.record(s)
        b.synchronize()
        one = max(a.elapsed_time(b), 1e-3)
        for _ in range(int(warm_ms / one) + 1):
            g.replay()
        a.record(s)
        for _ in range(reps):
            g.replay()
        b.record(s)
    b.synchronize()
    ms = a.elapsed_time(b) / (reps * n)
    del g
    return ms


def graph_time_ms(fn, n, torch, reps=3):
    """Average ms per call of fn over n calls captured into one HIP graph and
    replayed (removes host launch gaps for microsecond kernels).  Returns None
    if capture is not possible."""
    s = torch.cuda.Stream()
    try:
        with torch.cuda.stream(s):
            fn()
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=s):
            for _ in range(n):
                fn()
        g.replay()
        torch.cuda.synchronize()
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        with torch.cuda.stream(s):
            a.record(s)
            for _ in range(reps):
                g.replay()
            b.record(s)
        b.synchronize()
        ms = a.elapsed_time(b) / (reps * n)
        del g
        return ms
    except Exception:
        torch.cuda.synchronize()
        return None


PARTIAL_ROWS = 1024  # lx_dit.cpp kPartialRows


def dit_projection_plan(rows, N):
    """How the estimator runs a block projection (lx_dit.cpp, forward_core): the
    split-operand GEMM with fragment-order weights on 64-row tiles; up to 1024
    rows the out / FF2 projections (N = D) as two K slices whose sum is folded
    into the next modulated LayerNorm.  Returns (kind, slices)."""
    if N == 1024 and rows <= PARTIAL_ROWS:
        return "partial", 2
    return "direct", 1


def split_tail_fits(rows, N, cus):
    """Whether lx_linear_bx's split tail engages for a 64-row-tile launch (the
    estimator asks for it on the QKV projection): tile count between CUs and
    2 CUs with (tiles - CUs) * S = CUs for S = 2 or 4."""
    tiles = -(-rows // 64) * (N // 128)
    return any(cus < tiles and (tiles - cus) * s == cus for s in (2, 4))


def gemm_kernels(torch, ops, T, dev):
    """Per-class timings of one estimator block's launches at the step's shapes,
    each class on the kernel and plan the estimator runs for it (the split-operand
    GEMM with fragment-order weights, 64-row tiles; out / FF2 as two K slices at
    B*T <= 1024 rows, their sum folded into the next LayerNorm, which is timed as
    its own class), with the fp32 matrix-core GEMM and hipBLASLt on the same
    shapes for reference."""
    D, F, B = 1024, 2048, 2
    M = B * T
    g = torch.Generator(device=dev).manual_seed(3)
    xd = torch.randn(M, D, device=dev, generator=g)      # contiguous, as the estimator's xn / att
    xf = torch.randn(M, F, device=dev, generator=g)      # contiguous, as the GELU output
    wq = torch.randn(3 * D, D, device=dev, generator=g) * 0.02
    w1 = torch.randn(F, D, device=dev, generator=g) * 0.02
    w2 = torch.randn(D, F, device=dev, generator=g) * 0.02
    wo = torch.randn(D, D, device=dev, generator=g) * 0.02
    bq = torch.zeros(3 * D, device=dev)
    b1 = torch.zeros(F, device=dev)
    bd = torch.zeros(D, device=dev)
    h = torch.randn(B, T, D, device=dev, generator=g)
    emb = torch.randn(B, 6 * D, device=dev, generator=g) * 0.1
    gate = emb[:, 2 * D:3 * D]
    pos = torch.arange(T, dtype=torch.int32, device=dev)
    qkv = torch.randn(M, 3 * D, device=dev, generator=g)
    att = torch.empty(B, T, D, device=dev)
    ff = torch.empty(M, F, device=dev)
    part = torch.empty(2, M, D, device=dev)
    xn = torch.empty(B, T, D, device=dev)
    rope = ops.Epilogue(kind=ops.LX_EPI_ROPE_PARTIAL, rows_per_batch=T, pos=pos.data_ptr(),
                        rot_dim=64, rope_section=D, rope_sections=2, rope_base=10000.0)
    gelu = ops.Epilogue(kind=ops.LX_EPI_GELU_TANH)
    gated = ops.Epilogue(kind=ops.LX_EPI_GATED_RESID, rows_per_batch=T, gate=gate.data_ptr(),
                         gate_stride=emb.stride(0))
    out = {}
    qv = qkv.view(B, T, 3 * D)
    hv = h.view(M, D)

    cus = torch.cuda.get_device_properties(dev).multi_processor_count
    scr = ops.bx_scratch(dev, bm=64)

    def proj(x, W, b, ep, y, pack_out=False, pack_from=0, split_tail=True):
        N = W.shape[0]
        wf = ops.wfrag_pack(W)
        kind, sl = dit_projection_plan(M, N)
        fp32 = (lambda: ops.linear(x, W, b, ep, out=y))
        xp = pack2(torch, x)
        st = dict(scratch=scr, split_tail=True) if split_tail else {}

        def bx(products):
            # with three products the estimator passes its activations as
            # two-part packed rows (and FF0 writes its output that way)
            pk = products == 3
            a = xp if pk else x
            if kind == "partial":
                return lambda: ops.linear_bx(a, wf, N, out=part, out_kind=ops.LX_BX_OUT_PARTIAL,
                                             bm=64, slices=sl, products=products, a_packed=pk)
            ok = ops.LX_BX_OUT_PACKED if pk and pack_out else ops.LX_BX_OUT_F32
            pf = pack_from if pk and pack_out else 0
            return lambda: ops.linear_bx(a, wf, N, b, ep, out=y, out_kind=ok, bm=64,
                                         products=products, a_packed=pk, pack_from=pf, **st)
        kern = (f"gemm_bx_kernel 64x128, {DIT_PRODUCTS} products"
                + (", packed activations" if DIT_PRODUCTS == 3 else "")
                + (f", {sl} K slices (sum folded into adaln_resid)" if kind == "partial" else "")
                + (", split tail" if split_tail and split_tail_fits(M, N, cus) else ""))
        return bx(DIT_PRODUCTS), kern, fp32, bx(6)
    cases = {
        # q fp32, k and v packed for the split attention (T = 500's layout)
        "gemm_qkv_rope": (proj(xd, wq, bq, rope, qkv, pack_out=True, pack_from=D),
                          2 * M * 3 * D * D, 1),
        "gemm_out_gated": (proj(xd, wo, bd, gated, hv), 2 * M * D * D, 1),
        "gemm_ff0_gelu": (proj(xd, w1, b1, gelu, ff, pack_out=True), 2 * M * F * D, 1),
        "gemm_ff2_gated": (proj(xf, w2, bd, gated, hv), 2 * M * D * F, 1),
        "attention": ((lambda: ops.attention(qv[..., :D], qv[..., D:2 * D], qv[..., 2 * D:], 16,
                                             out=att, products=DIT_PRODUCTS,
                                             out_packed=DIT_PRODUCTS == 3,
                                             kv_packed=DIT_PRODUCTS == 3),
                       f"attn_bx_kernel ({DIT_PRODUCTS} products) / attn_flash_kernel", None,
                       lambda: ops.attention(qv[..., :D], qv[..., D:2 * D], qv[..., 2 * D:], 16,
                                             out=att, products=6)),
                      4 * B * 16 * T * T * 64, 1),
    }
    # hipBLASLt (torch.mm, fp32) on the same plain-GEMM shapes, as a library reference point
    lib_ref = {
        "gemm_qkv_rope": lambda: torch.mm(xd, wq.T),
        "gemm_out_gated": lambda: torch.mm(xd, wo.T),
        "gemm_ff0_gelu": lambda: torch.mm(xd, w1.T),
        "gemm_ff2_gated": lambda: torch.mm(xf, w2.T),
    }
    for name, ((fn, kern, fp32_fn, six_fn), flops, per_block) in cases.items():
        ms = steady_launch_ms(fn, torch)
        out[name] = {"avg_us": ms * 1e3, "flop": flops, "tflops": flops / (ms * 1e-3) / 1e12,
                     "per_block": per_block, "kernel": kern}
        if fp32_fn is not None:  # the fp32 kernel on the same class, for comparison
            out[name]["fp32_kernel_us"] = steady_launch_ms(fp32_fn, torch) * 1e3
        if six_fn is not None:  # the six-product split on the same class
            out[name]["six_products_us"] = steady_launch_ms(six_fn, torch) * 1e3
        if name in lib_ref:
            try:
                out[name]["hipblaslt_us"] = steady_launch_ms(lib_ref[name], torch) * 1e3
            except RuntimeError:  # library call not capturable: no reference figure
                torch.cuda.synchronize()
    # the modulated LayerNorms of a block (two per block): at <= 1024 rows each
    # folds the previous projection's two K slices into h first
    if dit_projection_plan(M, D)[0] == "partial":
        ms = steady_launch_ms(lambda: ops.adaln_resid(h, part, bd, gate, emb[:, :D],
                                                      emb[:, D:2 * D], out=xn,
                                                      packed=DIT_PRODUCTS == 3), torch)
        nbytes = 5 * M * D * 4 + 4 * B * D * 4
        kern = "adaln_resid_kernel (2 K slices + bias, gated residual, LayerNorm)"
    else:
        ms = steady_launch_ms(lambda: ops.ada_ln(h, emb[:, D:2 * D], emb[:, :D], out=xn), torch)
        nbytes = 2 * M * D * 4 + 2 * B * D * 4
        kern = "adaln_kernel"
    out["adaln"] = {"avg_us": ms * 1e3, "flop": 0, "tflops": 0.0, "per_block": 2, "kernel": kern,
                    "gbs": nbytes / (ms * 1e-3) / 1e9, "bytes": nbytes}
    return out


def fused_ops_gbs(torch, ops, dev):
    """Achieved HBM GB/s per fused op: algorithmic bytes (each tensor read once,
    output written once) / HIP-event time per launch, each launch on its own
    buffer set so the working set (> 256 MB) streams from HBM."""
    res = {}
    g = torch.Generator(device=dev).manual_seed(9)
    ROT = 320 * 2**20  # bytes cycled through per op

    def timed(make, call, set_bytes):
        nset = max(2, int(ROT // set_bytes))
        sets = [make() for _ in range(nset)]
        it = [0]

        def fn():
            call(*sets[it[0] % nset])
            it[0] += 1
        ms = graph_time_ms(fn, nset, torch)
        how = "graph"
        if ms is None:
            ms, how = event_time_ms(fn, nset, torch), "events"
        del sets
        return ms, how

    def run(name, make, call, algo_bytes, set_bytes, shape_note):
        ms, how = timed(make, call, set_bytes)
        # the same bytes moved by a plain device-to-device copy (half read, half
        # written), same rotation and timing: the practical streaming ceiling
        # for a kernel of this size on this device
        half = max(4, int(algo_bytes) // 8)
        cms, _ = timed(lambda: (torch.empty(half, device=dev), torch.empty(half, device=dev)),
                       lambda a, b: b.copy_(a), 8 * half)
        gbs = algo_bytes / (ms * 1e-3) / 1e9
        copy_gbs = 8 * half / (cms * 1e-3) / 1e9
        res[name] = {"shape": shape_note, "bytes": int(algo_bytes), "avg_us": ms * 1e3,
                     "timing": how, "gbs": gbs, "frac": gbs / HBM_PEAK_GBS,
                     "copy_same_bytes_us": cms * 1e3, "copy_gbs": copy_gbs,
                     "frac_of_copy": gbs / copy_gbs}

    for T in (500, 3000):
        B, D = 2, 1024
        N = B * T
        emb = torch.randn(B, 6 * D, device=dev, generator=g) * 0.1
        run(f"adaln_T{T}",
            lambda: (torch.randn(B, T, D, device=dev, generator=g), torch.empty(B, T, D, device=dev)),
            lambda x, y: ops.ada_ln(x, emb[:, D:2 * D], emb[:, :D], out=y),
            2 * N * D * 4 + 2 * B * D * 4, 2 * N * D * 4, f"B={B} T={T} D={D}")
        run(f"adaln_resid_T{T}",
            lambda: (torch.randn(B, T, D, device=dev, generator=g),
                     torch.randn(2, N, D, device=dev, generator=g),
                     torch.empty(B, T, D, device=dev)),
            lambda hh, pp, y: ops.adaln_resid(hh, pp, None, emb[:, 2 * D:3 * D], emb[:, :D],
                                              emb[:, D:2 * D], out=y),
            5 * N * D * 4 + 3 * B * D * 4, 5 * N * D * 4,
            f"B={B} T={T} D={D}, 2 K slices into h, then LayerNorm")
        run(f"gelu_T{T}",
            lambda: (torch.randn(N * 2048, device=dev, generator=g), torch.empty(N * 2048, device=dev)),
            lambda h, y: ops.gelu_tanh(h, out=y),
            2 * N * 2048 * 4, 2 * N * 2048 * 4, f"N={N} F=2048")
        run(f"gated_residual_T{T}",
            lambda: (torch.randn(B, T, D, device=dev, generator=g), torch.randn(B, T, D, device=dev, generator=g)),
            lambda x, y: ops.gated_residual(x, y, emb[:, 2 * D:3 * D]),
            3 * N * D * 4 + B * D * 4, 2 * N * D * 4, f"B={B} T={T} D={D}")
        pos = torch.arange(T, dtype=torch.int32, device=dev)
        run(f"rope_partial_T{T}",
            lambda: (torch.randn(B, T, D, device=dev, generator=g), torch.randn(B, T, D, device=dev, generator=g)),
            lambda q, k: ops.rope_partial(q, k, pos),
            2 * (2 * N * 64 * 4), 2 * N * D * 4, f"q,k B={B} T={T}, 64 of {D} channels")
    L, H, I = 256, 896, 4864
    wn = torch.randn(H, device=dev, generator=g)
    run("rmsnorm_L256",
        lambda: (torch.randn(L, H, device=dev, generator=g), torch.empty(L, H, device=dev)),
        lambda x, y: ops.rms_norm(x, wn, out=y), 2 * L * H * 4 + H * 4, 2 * L * H * 4, "L=256 H=896")
    posl = torch.arange(L, dtype=torch.int32, device=dev)
    # q (14 heads) and k (2 heads) are adjacent in the fused q|k|v row: one call
    run("rope_neox_L256",
        lambda: (torch.randn(L, 1152, device=dev, generator=g),),
        lambda qkv: ops.rope_full(qkv[:, :1024], posl, 16),
        2 * L * 1024 * 4, L * 1152 * 4, "q 14 + k 2 heads x 64, L=256")
    run("swiglu_L256",
        lambda: (torch.randn(L * I, device=dev, generator=g), torch.randn(L * I, device=dev, generator=g),
                 torch.empty(L * I, device=dev)),
        lambda a, b, c: ops.swiglu(a, b, out=c), 3 * L * I * 4, 3 * L * I * 4, "L=256 I=4864")
    table = torch.randn(151936, 896, device=dev, generator=g)
    ids = list(range(0, 151936, 151936 // 256))[:256]
    run("embed_gather_n256",
        lambda: (torch.empty(256, 896, device=dev),),
        lambda y: ops.embed_gather(table, ids, out=y), 2 * 256 * 896 * 4 + 256 * 4,
        256 * 896 * 4, "256 rows of the 151936x896 text table")
    return res


def copy_ceiling_gbs(torch, dev, mib=512, reps=10):
    """The device's practical streaming ceiling: a plain device-to-device copy
    (torch copy_) of `mib` MiB into a second buffer (2 x mib MiB moved per copy),
    timed with HIP events over `reps` copies after a warm-up."""
    n = mib * 2**20 // 4
    src = torch.ones(n, device=dev)
    dst = torch.empty_like(src)
    dst.copy_(src)
    torch.cuda.synchronize()
    s = torch.cuda.current_stream()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(s)
    for _ in range(reps):
        dst.copy_(src)
    e1.record(s)
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / reps
    gbs = 2 * n * 4 / (ms * 1e-3) / 1e9
    del src, dst
    return {"bytes_moved": 2 * n * 4, "avg_us": round(ms * 1e3, 2), "gbs": round(gbs, 1),
            "frac": round(gbs / HBM_PEAK_GBS, 4), "kernel": "torch copy_, device to device"}


def stream_ceiling_gbs(torch, ops, dev, mib=512, reps=10):
    """The library's own streaming ceiling: its tanh-GELU (a handful of VALU
    instructions per element, non-temporal float4 loads and stores) over a
    `mib` MiB input into a second buffer (2 x mib MiB moved per launch), HIP
    events over `reps` launches after a warm-up."""
    n = mib * 2**20 // 4
    src = torch.randn(n, device=dev)
    dst = torch.empty_like(src)
    ops.gelu_tanh(src, out=dst)
    torch.cuda.synchronize()
    s = torch.cuda.current_stream()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(s)
    for _ in range(reps):
        ops.gelu_tanh(src, out=dst)
    e1.record(s)
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / reps
    gbs = 2 * n * 4 / (ms * 1e-3) / 1e9
    del src, dst
    return {"bytes_moved": 2 * n * 4, "avg_us": round(ms * 1e3, 2), "gbs": round(gbs, 1),
            "frac": round(gbs / HBM_PEAK_GBS, 4),
            "kernel": "lx_gelu_tanh_f32 (gelu_kernel), non-temporal float4 stream"}


def long_utterance(torch, est, dev, g, steps=3, T=3000):
    """ms per CFG Euler step at T=3000 (the long-utterance config; T=1000 for the
    medium one), same estimator."""
    from larynx_amd.flow import cfm_t_span
    x = torch.randn(80, T, device=dev, generator=g)
    mu = torch.randn(80, T, device=dev, generator=g)
    cond = torch.randn(80, T, device=dev, generator=g)
    spks = torch.randn(80, device=dev, generator=g) / 80 ** 0.5
    ts = cfm_t_span(10)
    est.cfm_step(x, mu, cond, spks, float(ts[0]), float(ts[1] - ts[0]))
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(steps):
        est.cfm_step(x, mu, cond, spks, float(ts[i]), float(ts[i + 1] - ts[i]))
    torch.cuda.synchronize()
    ms = (time.perf_counter() - t0) * 1e3 / steps
    return {"T": T, "ms_per_step": round(ms, 3), "mel_frames_per_s": round(T / ms * 1e3, 1)}


def flow_infer(torch, dev, g, dit_params, n_prompt=50, n_tokens=200, prompt_frames=100):
    """Whole FlowDecoder::infer of a 10 s utterance (250 tokens -> 500 mel frames,
    100 prompt frames): frontend + 10 CFG Euler steps + output copy, host token
    ids in, mel frames past the prompt out."""
    from larynx_amd.flow import FlowDecoder, flow_frontend_param_shapes
    front = {n: torch.randn(*sh, device=dev, generator=g) * 0.02
             for n, sh in flow_frontend_param_shapes()}
    dec = FlowDecoder(front, dit_params, max_tokens=n_prompt + n_tokens)
    pt = torch.randint(0, 6561, (n_prompt,), generator=g, device=dev).cpu().tolist()
    tk = torch.randint(0, 6561, (n_tokens,), generator=g, device=dev).cpu().tolist()
    MT = 2 * (n_prompt + n_tokens)
    pf = torch.randn(prompt_frames, 80, device=dev, generator=g)
    spk = torch.randn(192, device=dev, generator=g)
    z = torch.randn(80, MT, device=dev, generator=g)
    dec.infer(pt, tk, pf, spk, z)
    torch.cuda.synchronize()
    n = 3
    t0 = time.perf_counter()
    for _ in range(n):
        dec.infer(pt, tk, pf, spk, z)
    torch.cuda.synchronize()
    ms = (time.perf_counter() - t0) * 1e3 / n
    dec.close()
    return {"tokens": n_prompt + n_tokens, "mel_frames": MT, "prompt_frames": prompt_frames,
            "ms": round(ms, 3), "out_mel_frames_per_s": round((MT - prompt_frames) / ms * 1e3, 1)}


def qwen2_lm(torch, dev, g):
    """Qwen2-0.5B (24 layers, full vocabularies): prefill at L=256 (160 text + 96
    speech-prompt rows) and single-token decode against KV caches of 1 / 256 / 1024 /
    2048 entries.  Decode is weight-streaming: 1.46 GB of weights per token."""
    from larynx_amd.llm import Qwen2Config, Qwen2LM, qwen2_param_shapes
    cfg = Qwen2Config()
    params = {n: torch.randn(*sh, device=dev, generator=g) * 0.02
              for n, sh in qwen2_param_shapes(cfg)}
    lm = Qwen2LM(params, cfg, max_ctx=2304)
    text = [int(v) for v in torch.randint(0, cfg.text_vocab, (160,), generator=g,
                                          device=dev).cpu()]
    speech = [int(v) for v in torch.randint(0, 6564, (94,), generator=g, device=dev).cpu()]
    lm_in = lm.build_lm_input(text, speech)
    lm.prefill(lm_in)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(3):
        lm.prefill(lm_in)
    torch.cuda.synchronize()
    prefill_ms = (time.perf_counter() - t0) * 1e3 / 3
    lm.set_products(6)  # the six-product split on the same prefill, for comparison
    lm.prefill(lm_in)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(3):
        lm.prefill(lm_in)
    torch.cuda.synchronize()
    six_ms = (time.perf_counter() - t0) * 1e3 / 3
    lm.set_products(3)
    out = {"prefill_L256_ms": round(prefill_ms, 3), "prefill_products": 3,
           "prefill_L256_ms_six_products": round(six_ms, 3), "decode_ms_per_token": {}}
    L, H, KVW = lm_in.shape[0], cfg.hidden, cfg.n_kv_heads * cfg.head_dim
    NQKV = H + 2 * KVW
    rec = profiled_kernels(torch, lambda: lm.prefill(lm_in))
    s_o = prefill_bx_slices(L, H, H)
    s_d = prefill_bx_slices(L, H, cfg.intermediate)
    s_q = prefill_bx_slices(L, NQKV, H)
    # o_proj and down_proj reduce passes alternate within a layer
    rr = [(s + 3) * L * H * 4 + H * 4 for s in (s_o, s_d)]
    out["in_path"] = {
        "resid_rmsnorm_prefill": kernel_gbs(
            rec, "resid_rmsnorm_kernel", rr,
            f"L={L}: {s_o} (o_proj) / {s_d} (down_proj) K slices + residual, next RMSNorm"),
        "qkv_rope_cache_prefill": kernel_gbs(
            rec, "qkv_rope_cache_kernel", (s_q + 1) * L * NQKV * 4 + NQKV * 4,
            f"L={L}: {s_q} K slices + bias, NEOX rotary, q out and K/V cache append"),
    }
    weight_bytes = sum(t.numel() for n, t in params.items() if n != "embed_tokens.weight") * 4
    out["decode_stream_gbs"] = {}
    for cache in (1, 256, 1024, 2048):
        lm.set_cache_len(cache)
        lm.decode(17)
        torch.cuda.synchronize()
        n = 20
        t0 = time.perf_counter()
        for i in range(n):
            lm.set_cache_len(cache)
            lm.decode(100 + i)
        torch.cuda.synchronize()
        ms = (time.perf_counter() - t0) * 1e3 / n
        out["decode_ms_per_token"][str(cache)] = round(ms, 4)
        # weights + the K/V rows attention reads (24 layers x 2 x (cache+1) x 128 floats)
        kv_bytes = cfg.n_layers * 2 * (cache + 1) * cfg.n_kv_heads * cfg.head_dim * 4
        out["decode_stream_gbs"][str(cache)] = round((weight_bytes + kv_bytes) / (ms * 1e-3) / 1e9,
                                                     1)
    ms1 = out["decode_ms_per_token"]["1"]
    out["decode_weight_stream_gbs_at_cache1"] = round(weight_bytes / (ms1 * 1e-3) / 1e9, 1)
    lm.close()
    del params
    return out


def cpu_baseline(T, seconds):
    """The reference's CPU path for the same step: its ggml graph for one CFG
    Euler step (22-block DiT, B=2, T) restated node by node in fp32, timed on
    this host's cores (oracle/lx_ggml_cpu.c; ggml itself is absent).  One
    warm-up step, then the median of at least five steps (more while under
    `seconds`)."""
    import numpy as np
    from oracle import oracle as orc
    from oracle import ggml_cpu
    from larynx_amd.flow import DiTConfig, dit_param_shapes
    params = orc.make_params(dit_param_shapes(DiTConfig()), 1)
    g = ggml_cpu.GgmlCpuDit(params, B=2, max_T=T)
    x = orc.normal((80, T), 2, 1)
    mu2, cond2, spks2 = g.cfm_inputs(orc.normal((80, T), 2, 2), orc.normal((80, T), 2, 3),
                                     orc.normal((80,), 2, 4, 1.0 / np.sqrt(80.0)))
    g.cfm_step(x, mu2, cond2, spks2, 0.0, 0.0123)  # warm-up (page in weights, threads)
    times = []
    t_start = time.perf_counter()
    while True:
        t0 = time.perf_counter()
        g.cfm_step(x, mu2, cond2, spks2, 0.0123, 0.05)
        times.append(time.perf_counter() - t0)
        if len(times) >= 5 and (time.perf_counter() - t_start > seconds or len(times) >= 20):
            break
    g.close()
    t_step = float(np.median(times))
    try:
        affinity = len(os.sched_getaffinity(0))
    except AttributeError:
        affinity = os.cpu_count()
    return {"value": T / t_step, "unit": "mel frames/s", "cores": ggml_cpu.threads(),
            "kind": "port",
            "name": "ggml-equivalent CPU restatement (ggml unavailable offline)",
            "cpu_model": ggml_cpu.cpu_model(), "nproc": affinity, "isa": ggml_cpu.isa(),
            "ms_per_step": round(t_step * 1e3, 1),
            "sample": f"{len(times)} CFG Euler steps of the 22-block DiT at B=2, T={T} through "
                      f"the reference's fp32 ggml node graph (one pass per node, KQ "
                      f"materialised, blocked SGEMM), median {t_step:.3f} s/step, "
                      f"{ggml_cpu.threads()} OpenMP threads"}


TRAFFIC_PROFILE = os.path.join(ROOT, "profiles", "gemm_bx_qkv_rope_T500_traffic.md")
COPY_PROBE_BYTES = 256 << 20


def counter_probe(torch, ops, launches=20):
    """The DiT step's matrix kernels at T=500, each `launches` times on its own,
    as the step runs them: the QKV projection with the rotary epilogue (M=1000,
    N=3072, K=1024) and FF0 with the GELU epilogue (N=2048) on the split-operand
    GEMM with fragment-order weights (64-row tiles), the out (K=1024) and FF2
    (K=2048) projections as two K slices each, and the 16-head attention (B=2,
    T=500): the workload of the rocprofv3 --pmc passes whose readings
    (matrix-core busy, VALU and LDS activity) are summarised per kernel."""
    dev = torch.device("cuda:0")
    D, T, B, F = 1024, 500, 2, 2048
    M = B * T
    g = torch.Generator(device=dev).manual_seed(4)
    xd = torch.randn(M, D, device=dev, generator=g)
    wq = torch.randn(3 * D, D, device=dev, generator=g) * 0.02
    bq = torch.zeros(3 * D, device=dev)
    w0 = torch.randn(F, D, device=dev, generator=g) * 0.02
    b0 = torch.zeros(F, device=dev)
    pos = torch.arange(T, dtype=torch.int32, device=dev)
    qkv = torch.empty(M, 3 * D, device=dev)
    ff = torch.empty(M, F, device=dev)
    att = torch.empty(B, T, D, device=dev)
    rope = ops.Epilogue(kind=ops.LX_EPI_ROPE_PARTIAL, rows_per_batch=T, pos=pos.data_ptr(),
                        rot_dim=64, rope_section=D, rope_sections=2, rope_base=10000.0)
    gelu = ops.Epilogue(kind=ops.LX_EPI_GELU_TANH)
    q3 = qkv.view(B, T, 3 * D)
    wo = torch.randn(D, D, device=dev, generator=g) * 0.02
    w2 = torch.randn(D, F, device=dev, generator=g) * 0.02
    fq, f0, fo, f2 = (ops.wfrag_pack(w) for w in (wq, w0, wo, w2))
    part = torch.empty(2, M, D, device=dev)
    # as the estimator runs them: with three products the activations arrive
    # as two-part packed rows and FF0 / attention write theirs packed
    pk = DIT_PRODUCTS == 3
    xa = pack2(torch, xd) if pk else xd
    ff0_out = ops.LX_BX_OUT_PACKED if pk else ops.LX_BX_OUT_F32
    scr = ops.bx_scratch(dev, bm=64)  # the QKV projection's split tail, as in the step
    torch.cuda.synchronize()
    for _ in range(launches):
        ops.linear_bx(xa, fq, 3 * D, bq, rope, out=qkv, out_kind=ff0_out, bm=64,
                      products=DIT_PRODUCTS, a_packed=pk, pack_from=D if pk else 0,
                      scratch=scr, split_tail=True)
    for _ in range(launches):
        ops.linear_bx(xa, f0, F, b0, gelu, out=ff, out_kind=ff0_out, bm=64,
                      products=DIT_PRODUCTS, a_packed=pk)
    for _ in range(launches):
        ops.linear_bx(xa, fo, D, out=part, out_kind=ops.LX_BX_OUT_PARTIAL, bm=64, slices=2,
                      products=DIT_PRODUCTS, a_packed=pk)
    for _ in range(launches):
        ops.linear_bx(ff, f2, D, out=part, out_kind=ops.LX_BX_OUT_PARTIAL, bm=64, slices=2,
                      products=DIT_PRODUCTS, a_packed=pk)
    for _ in range(launches):
        ops.attention(q3[..., :D], q3[..., D:2 * D], q3[..., 2 * D:], 16, 16, out=att,
                      products=DIT_PRODUCTS, out_packed=pk, kv_packed=pk)
    torch.cuda.synchronize()
    print(f"counter probe: {launches} x QKV, FF0, out, FF2 GEMMs and attention (B={B} T={T})",
          flush=True)


def prefill_probe(torch, runs=10):
    """The Qwen2-0.5B prefill at L=256 (full 24-layer model, random N(0, 0.02)
    weights) `runs` times on its own: the workload of the rocprofv3 --pmc
    passes whose readings (clock, matrix-core busy, HBM fetch) are summarised
    per prefill kernel."""
    from larynx_amd.llm import Qwen2Config, Qwen2LM, qwen2_param_shapes
    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev).manual_seed(5)
    cfg = Qwen2Config()
    params = {n: torch.randn(*sh, device=dev, generator=g) * 0.02
              for n, sh in qwen2_param_shapes(cfg)}
    lm = Qwen2LM(params, cfg, max_ctx=2304)
    lm_in = lm.build_lm_input(list(range(100, 260)), list(range(10, 104)))
    torch.cuda.synchronize()
    for _ in range(runs):
        lm.prefill(lm_in)
    torch.cuda.synchronize()
    lm.close()
    print(f"prefill probe: {runs} x Qwen2 prefill (L={lm_in.shape[0]})", flush=True)


def traffic_probe(torch, ops, launches=20):
    """Launch the QKV projection as the step runs it (split-operand GEMM with
    fragment-order weights, 64-row tiles; B*T = 1000, N = 3072, K = 1024, rotary
    epilogue) and a plain
    256 MiB device-to-device copy, each `launches` times, with nothing else on
    the device: the workload of the two rocprofv3 --pmc
    runs (FETCH_SIZE, then WRITE_SIZE) whose per-dispatch readings give the
    dominant kernel's HBM traffic, scaled by the copy's reading for its known
    size."""
    dev = torch.device("cuda:0")
    D, T, B = 1024, 500, 2
    M = B * T
    g = torch.Generator(device=dev).manual_seed(3)
    xd = torch.randn(M, D, device=dev, generator=g)
    wq = torch.randn(3 * D, D, device=dev, generator=g) * 0.02
    bq = torch.zeros(3 * D, device=dev)
    pos = torch.arange(T, dtype=torch.int32, device=dev)
    qkv = torch.empty(M, 3 * D, device=dev)
    rope = ops.Epilogue(kind=ops.LX_EPI_ROPE_PARTIAL, rows_per_batch=T, pos=pos.data_ptr(),
                        rot_dim=64, rope_section=D, rope_sections=2, rope_base=10000.0)
    src = torch.randn(COPY_PROBE_BYTES // 4, device=dev, generator=g)
    dst = torch.empty_like(src)
    fq = ops.wfrag_pack(wq)
    pk = DIT_PRODUCTS == 3  # the estimator's packed activations
    xa = pack2(torch, xd) if pk else xd
    scr = ops.bx_scratch(dev, bm=64)  # the split tail, as in the step
    torch.cuda.synchronize()
    for _ in range(launches):
        ops.linear_bx(xa, fq, 3 * D, bq, rope, out=qkv, bm=64, products=DIT_PRODUCTS,
                      a_packed=pk, pack_from=D if pk else 0,
                      out_kind=ops.LX_BX_OUT_PACKED if pk else ops.LX_BX_OUT_F32,
                      scratch=scr, split_tail=True)
    torch.cuda.synchronize()
    for _ in range(launches):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(f"traffic probe: {launches} x QKV GEMM (M={M} N={3 * D} K={D}), "
          f"{launches} x copy of {COPY_PROBE_BYTES} bytes", flush=True)


def committed_traffic():
    """HBM bytes per launch of the dominant kernel, from the committed summary
    of the two --pmc runs over --traffic-probe (None when it is absent)."""
    try:
        with open(TRAFFIC_PROFILE) as f:
            for ln in f:
                if ln.startswith("traffic_bytes_per_launch:"):
                    return int(ln.split(":", 1)[1].strip())
    except OSError:
        pass
    return None


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (requested --gpus {args.gpus}); the DiT path "
              "shards by CFG row / heads across GPUs by design but no multi-GPU figure is "
              "produced.", file=sys.stderr)
        sys.exit(2)
    import torch
    if not torch.cuda.is_available():
        print("bench.py needs a HIP device", file=sys.stderr)
        sys.exit(1)
    from larynx_amd import ops
    from larynx_amd.flow import DiTConfig, DiTEstimator, cfm_t_span, dit_param_shapes
    if args.traffic_probe:
        traffic_probe(torch, ops)
        return
    if args.counter_probe:
        counter_probe(torch, ops)
        return
    if args.prefill_probe:
        prefill_probe(torch)
        return

    dev = torch.device("cuda:0")
    T = args.T
    cfg = DiTConfig()
    g = torch.Generator(device=dev).manual_seed(0)
    params = {}
    for name, shape in dit_param_shapes(cfg):
        params[name] = torch.randn(*shape, device=dev, generator=g) * 0.02
    est = DiTEstimator(params, cfg, B=2, max_T=max(T, 3000))
    dit_params = params
    x = torch.randn(80, T, device=dev, generator=g)
    mu = torch.randn(80, T, device=dev, generator=g)
    cond = torch.randn(80, T, device=dev, generator=g)
    spks = torch.randn(80, device=dev, generator=g) / 80 ** 0.5
    ts = cfm_t_span(cfg.n_timesteps)
    sched = [(float(ts[i]), float(ts[i + 1] - ts[i])) for i in range(cfg.n_timesteps)]

    n_sched = len(sched)
    z = torch.randn(80, T, device=dev, generator=g)

    def step(i):
        t, dt = sched[i % n_sched]
        est.cfm_step(x, mu, cond, spks, t, dt)

    def run_steps(k):
        # k Euler steps as the reference's CFM loop runs them: whole 10-step
        # solves (one stacked modulation GEMV per solve), the remainder as
        # single steps
        for _ in range(k // n_sched):
            est.cfm_solve(z, mu, cond, spks)
        for i in range(k % n_sched):
            step(i)

    run_steps(args.warmup)
    torch.cuda.synchronize()
    s = torch.cuda.current_stream()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    e0.record(s)
    run_steps(args.steps)
    e1.record(s)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ev_ms = e0.elapsed_time(e1)
    ms_per_step = wall * 1e3 / args.steps
    value = T * args.steps / wall

    # the same timed steps with the six-product projections (fp32-GEMM error level)
    est.set_products(6)
    run_steps(args.warmup)
    torch.cuda.synchronize()
    t6 = time.perf_counter()
    run_steps(args.steps)
    torch.cuda.synchronize()
    six_ms_per_step = (time.perf_counter() - t6) * 1e3 / args.steps
    est.set_products(DIT_PRODUCTS)

    # one 10-step solve (the reference's whole CFM loop), and 10 single steps
    # (each with its own time MLP and modulation GEMV), at the same shape
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    est.cfm_solve(z, mu, cond, spks)
    torch.cuda.synchronize()
    solve_ms = (time.perf_counter() - t1) * 1e3
    t1 = time.perf_counter()
    for i in range(n_sched):
        step(i)
    torch.cuda.synchronize()
    single_step_ms = (time.perf_counter() - t1) * 1e3 / n_sched

    # fused kernels as the step launches them (inputs just written by the
    # producing GEMM, as in the real step), from the runtime's activity records
    rec = profiled_kernels(torch, lambda: [step(i) for i in range(3)])
    rows, D, mel = 2 * T, 1024, 80
    p_slices = splitk_slices(rows, mel, D)
    # every modulated LayerNorm of the step runs as adaln_resid_kernel: the first
    # (block 0's) without slices, the other 2 * depth fold the previous
    # projection's two K slices into h first
    ln_plain = 2 * rows * D * 4 + 2 * 2 * D * 4
    ln_fold = 5 * rows * D * 4 + 4 * 2 * D * 4
    in_path = {
        "adaln_resid_in_step": kernel_gbs(
            rec, "adaln_resid_kernel", [ln_plain] + [ln_fold] * (2 * cfg.depth),
            f"the modulated LayerNorms of a step (B=2 T={T}): the first on h alone, the "
            f"other {2 * cfg.depth} after the out / FF2 projection's two K slices + bias into h "
            f"(gated residual)"),
        "euler_in_step": kernel_gbs(rec, "euler_kernel",
                                    p_slices * rows * mel * 4 + 2 * mel * T * 4 + mel * 4,
                                    f"{p_slices} proj_out K slices + bias summed, CFG "
                                    f"combine, x update (80 x {T})"),
    }

    kernels = gemm_kernels(torch, ops, T, dev)
    # the same classes as the step runs them: average duration of their launches
    # inside the three profiled Euler steps (activity records; under an external
    # profiler such as rocprofv3 these records are not meaningful)
    in_step = in_step_matrix(rec, ops)
    for k, v in in_step.items():
        if k in kernels and v:
            kernels[k]["in_step_us"] = v["avg_us"]
    # dominant kernel: largest share of a step among the matrix kernels (22
    # blocks, one launch each); its duration from the graph-replayed launches
    # (HIP events on the replay stream), the in-step average beside it
    dom_name, dom = max(((k, v) for k, v in kernels.items() if v["flop"]),
                        key=lambda kv: kv[1]["avg_us"] * kv[1]["per_block"])
    dom_us = dom["avg_us"]
    dom_tflops = dom["flop"] / (dom_us * 1e-6) / 1e12
    # MFMA utilisation: the GEMM's fp32 flops per second against the 157.3
    # TFLOP/s fp32 matrix peak, whatever pipe runs it
    roofline = {"kernel": dom_name, "impl": dom["kernel"], "bound": "mfma",
                "achieved": round(dom_tflops, 3), "peak": MFMA_F32_PEAK_TFLOPS,
                "unit": "TFLOP/s", "frac": round(dom_tflops / MFMA_F32_PEAK_TFLOPS, 4),
                "traffic": (committed_traffic()
                            if dom_name == "gemm_qkv_rope" and T == 500 else None),
                "avg_us": round(dom_us, 2), "flop_per_launch": dom["flop"],
                "timing": "graph-replayed launches, HIP events on the replay stream",
                "in_step_us": (round(dom["in_step_us"], 2) if "in_step_us" in dom else None)}
    if dom["kernel"].startswith(("gemm_bx_kernel", "attn_bx_kernel")):
        # the same work as executed: bf16 MFMA products per fp32 product, against
        # the dense bf16 peak
        npr = DIT_PRODUCTS
        bf = npr * dom_tflops
        roofline["bf16_pipe"] = {"achieved": round(bf, 3), "peak": MFMA_BF16_PEAK_TFLOPS,
                                 "frac": round(bf / MFMA_BF16_PEAK_TFLOPS, 4),
                                 "note": f"{npr} bf16 MFMA products per fp32 product"}
    if "fp32_kernel_us" in dom:  # the fp32 matrix-core GEMM on the same class, for reference
        f32 = dom["flop"] / (dom["fp32_kernel_us"] * 1e-6) / 1e12
        roofline["fp32_kernel"] = {"impl": "gemm_pipe_kernel",
                                   "avg_us": round(dom["fp32_kernel_us"], 2),
                                   "achieved": round(f32, 3), "peak": MFMA_F32_PEAK_TFLOPS,
                                   "frac": round(f32 / MFMA_F32_PEAK_TFLOPS, 4)}
    gemm_flop_step = 22 * sum(k["flop"] for k in kernels.values())
    long_t = long_utterance(torch, est, dev, g)
    long_t["T1000"] = long_utterance(torch, est, dev, g, steps=5, T=1000)
    flow = None if args.no_flow else flow_infer(torch, dev, g, dit_params)
    del dit_params, params
    fused = {} if args.no_fused else fused_ops_gbs(torch, ops, dev)
    copy_ceiling = copy_ceiling_gbs(torch, dev)
    stream = stream_ceiling_gbs(torch, ops, dev)
    est.close()
    qwen = None if args.no_llm else qwen2_lm(torch, dev, g)

    cpu = None
    if not args.no_cpu:
        cpu = cpu_baseline(T, args.cpu_seconds)

    line = {
        "metric": "DiT Euler-step mel frames/s at T=500 B=2",
        "value": round(value, 1),
        "unit": "mel frames/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (random ~N(0,0.02) weights, N(0,1) mel inputs)",
        "config": {"workload": "CosyVoice3 Flow DiT estimator, CFG Euler steps of the "
                               "10-step CFM solve (22 blocks, dim 1024, 16x64 heads, ff 2048, "
                               "mel 80)",
                   "B": 2, "T": T, "blocks": 22, "cfg_rate": 0.7},
        "event_ms_per_step": round(ev_ms / args.steps, 4),
        "euler_10step_ms": round(solve_ms, 3),
        "single_step_ms": round(single_step_ms, 4),
        "step_tflops": round(gemm_flop_step / (ms_per_step * 1e-3) / 1e12, 2),
        "roofline": roofline,
        "products": DIT_PRODUCTS,
        "six_products": {"ms_per_step": round(six_ms_per_step, 4),
                         "value": round(T / (six_ms_per_step * 1e-3), 1),
                         "note": "same steps, block projections and attention as six bf16 "
                                 "products per fp32 product (fp32-GEMM error level)"},
        "kernels": {k: {kk: (round(vv, 2) if kk != "kernel" else vv)
                        for kk, vv in v.items() if kk in
                        ("avg_us", "in_step_us", "tflops", "hipblaslt_us", "kernel",
                         "fp32_kernel_us", "gbs", "six_products_us")}
                    for k, v in kernels.items()},
        "matrix_in_step": {k: ({"launches": v["launches"], "avg_us": round(v["avg_us"], 2)}
                               if v else None) for k, v in in_step.items()},
        "long_utterance": long_t,
        "flow_infer": flow,
        "qwen2": qwen,
        "fused_ops": {k: {kk: (round(vv, 4) if isinstance(vv, float) else vv)
                          for kk, vv in v.items()} for k, v in fused.items()},
        "fused_in_path": dict(in_path, **(qwen["in_path"] if qwen else {})),
        "copy_ceiling": copy_ceiling,
        "stream_ceiling": stream,
        "cpu_baseline": cpu,
    }
    if cpu:
        line["gpu_over_cpu"] = round(value / cpu["value"], 1)
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
