"""Benchmark of the MI355X attention hot path (one JSON line on stdout).

Headline workload (value): BASELINE configs[1] — Bonsai-4B decode attention
over all 36 layers at ctx 4096, batch 1. One step = for each layer:
q_norm_rope (1 token) -> kv_writeback of row 4096 -> split-K decode
attention over 4097 rows, replayed from a HIP graph. Inputs are resident in
HBM; the 36 layers' caches (350 MB per step) exceed the 256 MB Infinity
Cache, so every step streams the KV cache from HBM.

value = algorithmic bytes per step / step time, with per layer
4097 rows x 2304 B (K+V: 2 x (128 qs + 4 x 4 B d)) + 16384 B (q in, out).

Also reported: decode at ctx 32768 (config 5, rotating over 8 layers),
prefill pp2048 (metric) and the 2048-on-2048 chunked prefill (config 4) in
TFLOP/s of unmasked QK^T + PV work, the Bonsai-4B per-layer Q1_0 decode
matvecs (fused normed q/k/v, o, fused normed gate/up, silu down) over 36
layers of distinct weights in GB/s, the prefill projections (Q8_0
quantize + Q1_0 x Q8_0 matmul) of a Bonsai-4B layer at 512 tokens in TOPS,
and the CPU oracle on a bounded sample.
"""
import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "bonsai-pot_amd"))
# The bench build of the library: the product library's kernels plus the
# measurement hooks (include/bonsai_pot_hip_bench.h) this script times beside
# them.
os.environ.setdefault("BONSAI_POT_HIP_LIB", os.path.join(ROOT, "bonsai-pot_amd", "lib", "libbonsai_pot_hip_bench.so"))

METRIC = "decode-attn HBM GB/s (%peak) ctx4K/32K; prefill-attn TFLOP/s (%MFMA) pp2048"
HBM_PEAK_GBS = 8000.0
F16_MFMA_PEAK_TFLOPS = 2500.0
I8_MFMA_PEAK_TOPS = 5000.0
KV_ROW_BYTES = 2 * 8 * (128 + 16)   # 2304 B per cache row: K + V, 8 KV heads, 128 qs + 4 f32 d
QO_BYTES = 2 * 32 * 128 * 2         # q in + out, f16


def decode_bytes(n_keys: int) -> int:
    return n_keys * KV_ROW_BYTES + QO_BYTES


def prefill_flops(m: int, pos: int, n_head=32, d=128) -> int:
    pairs = m * pos + m * (m + 1) // 2      # unmasked (query, key) pairs per head
    return 4 * d * n_head * pairs


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--no-graph", action="store_true", help="eager launches instead of a HIP graph")
    ap.add_argument("--skip-cpu", action="store_true")
    ap.add_argument("--only", choices=["decode4k", "decode32k", "prefill", "chunked", "matvec", "matmul", "copy"], default=None,
                    help="run only one workload (for profiling)")
    return ap.parse_args()


class Bench:
    def __init__(self, torch, n_layer, max_seq, m_tokens, seed=0):
        from bonsai_pot_amd import Model, layout
        self.torch = torch
        self.cfg = layout.Config(n_layer=n_layer)
        cfg = self.cfg
        self.model = Model(cfg, max_seq)
        self.stream = torch.cuda.current_stream()
        self.model.set_stream(self.stream.cuda_stream)
        g = torch.Generator(device="cuda").manual_seed(seed)
        self.m = m_tokens
        # act: q [m, 4096] | k_cur [m, 1024] | v_cur [m, 1024] | out [m, 4096]
        self.q_off = 0
        self.k_off = m_tokens * cfg.q_dim
        self.v_off = self.k_off + m_tokens * cfg.kv_dim
        self.out_off = self.v_off + m_tokens * cfg.kv_dim
        n = self.out_off + m_tokens * cfg.q_dim
        self.act = torch.randn(n, generator=g, device="cuda", dtype=torch.float32).to(torch.float16)
        self.w = torch.ones(2 * cfg.head_dim, device="cuda", dtype=torch.float16)
        self.a, self.wp = self.act.data_ptr(), self.w.data_ptr()

    def fill_cache(self, rows: int, layers=None, seed=1):
        """Writes cache rows [0, rows) of each layer with kv_writeback of random K/V."""
        torch = self.torch
        cfg = self.cfg
        g = torch.Generator(device="cuda").manual_seed(seed)
        chunk = 4096
        buf = torch.empty(2 * chunk * cfg.kv_dim, device="cuda", dtype=torch.float16)
        for il in (range(cfg.n_layer) if layers is None else layers):
            for r0 in range(0, rows, chunk):
                n = min(chunk, rows - r0)
                buf.copy_(torch.randn(buf.numel(), generator=g, device="cuda").to(torch.float16))
                self.model.dispatch_kv_writeback_fused(buf.data_ptr(), self.wp, 0, chunk * cfg.kv_dim,
                                                       cfg.head_dim, il, r0, n)
        torch.cuda.synchronize()


def time_region(torch, fn, steps, warmup):
    """Seconds per fn() over `steps` calls after `warmup`, bracketed by
    synchronizations and timed with HIP events recorded on the current stream
    (the stream graph replays and the model's launches run on)."""
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(steps):
        fn()
    end.record()
    torch.cuda.synchronize()
    return start.elapsed_time(end) * 1e-3 / steps


def per_launch_us(torch, b, launch, n_launch, replays=5, warm_s=0.03):
    """Average device time of one launch: n_launch launches (rotating layers) are
    captured in a HIP graph and replayed between two HIP events recorded on the
    stream the kernels run on, so host launch latency is excluded (inter-kernel
    gaps of graph dispatch are included). The graph is first replayed for
    warm_s seconds, so that the timed replays run at the clocks of sustained
    load (a cold start measured up to 14 % slower)."""
    g = make_graph(torch, b, lambda: [launch(i) for i in range(n_launch)])
    t_end = time.perf_counter() + warm_s
    while True:
        g.replay()
        torch.cuda.synchronize()
        if time.perf_counter() >= t_end:
            break
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(replays):
        g.replay()
    end.record()
    torch.cuda.synchronize()
    return start.elapsed_time(end) * 1e3 / (replays * n_launch)


def run_decode_step(b: "Bench", pos: int, layers):
    """One decode step over `layers`: per layer q_norm_rope + kv_writeback of row
    `pos` + attention over rows [0, pos], as the fused two-launch entry point."""
    m = b.model
    for il in layers:
        m.dispatch_attention_decode_step(b.a, b.wp, b.q_off, b.k_off, b.v_off, b.out_off, 0, 128, il, pos)


def run_decode_step_unfused(b: "Bench", pos: int, layers):
    """The same step as the reference's dispatch sequence (three entry points)."""
    m = b.model
    for il in layers:
        m.dispatch_q_norm_rope_fused(b.a, b.wp, b.q_off, 0, pos, 1)
        m.dispatch_kv_writeback_fused(b.a, b.wp, b.k_off, b.v_off, 128, il, pos, 1)
        m.dispatch_attention_decode(b.a, b.q_off, b.out_off, il, pos)


def make_graph(torch, b, body):
    """Captures body() (launches on b.model's stream) into a HIP graph."""
    graph = torch.cuda.CUDAGraph()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    torch.cuda.synchronize()
    with torch.cuda.stream(side):
        b.model.set_stream(side.cuda_stream)
        body()                                   # warm-up outside capture
        torch.cuda.synchronize()
        with torch.cuda.graph(graph, stream=side):
            body()
    b.model.set_stream(torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    return graph


def bench_decode(torch, args, ctx, n_layer, graph_ok=True):
    pos = ctx                                    # step at pos attends pos + 1 rows
    b = Bench(torch, n_layer, pos + 1 + 63, 1, seed=ctx)
    b.fill_cache(pos, seed=ctx + 1)
    layers = list(range(n_layer))
    step_bytes = n_layer * decode_bytes(pos + 1)
    body = lambda: run_decode_step(b, pos, layers)
    eager_s = time_region(torch, body, max(3, args.steps // 5), 2)
    graph_s = None
    unfused_s = None
    if graph_ok and not args.no_graph:
        g = make_graph(torch, b, body)
        graph_s = time_region(torch, g.replay, args.steps, args.warmup)
        gu = make_graph(torch, b, lambda: run_decode_step_unfused(b, pos, layers))
        unfused_s = time_region(torch, gu.replay, args.steps, args.warmup)
    step_s = graph_s if graph_s is not None else eager_s
    # dominant kernel: decode attention alone, per launch, rotating layers
    n_l = 4 * n_layer
    avg_us = per_launch_us(
        torch, b, lambda i: b.model.dispatch_attention_decode(b.a, b.q_off, b.out_off, i % n_layer, pos), n_l)
    kbytes = decode_bytes(pos + 1)
    res = {
        "ctx": ctx, "n_keys": pos + 1, "layers": n_layer,
        "ms_per_step": step_s * 1e3, "ms_per_step_eager": eager_s * 1e3,
        "ms_per_step_graph": None if graph_s is None else graph_s * 1e3,
        "ms_per_step_graph_unfused": None if unfused_s is None else unfused_s * 1e3,
        "step_GBps": step_bytes / step_s / 1e9,
        "kernel_us_avg": avg_us,
        "kernel_bytes": kbytes, "kernel_GBps": kbytes / (avg_us * 1e-6) / 1e9,
    }
    res["kernel_frac_hbm"] = res["kernel_GBps"] / HBM_PEAK_GBS
    # The streaming-read floor of the same byte count on this GPU: the
    # library's plain read kernel (bp_debug_read_floor: every 16-byte word
    # read once, 4 loads in flight per thread, 512 workgroups: the fastest of
    # 512 / 1024 / 2048 / 4096 / 8192 on the box) over kbytes,
    # per launch in a graph, rotating over as many buffers as layers so that
    # (like the decode's rotating layers) the reads come from HBM, not the
    # 256 MB Infinity Cache. kernel_frac_of_read_floor = floor / (split +
    # merge time).
    from bonsai_pot_amd import lib as _lib
    nbytes16 = kbytes // 16 * 16
    rd = [torch.ones(nbytes16 // 4, device="cuda", dtype=torch.float32) for _ in range(n_layer)]
    sink = torch.zeros(1024, device="cuda", dtype=torch.int32)

    class _R:
        model = b.model

    def _read(i):
        rc = _lib.bp_debug_read_floor(rd[i % n_layer].data_ptr(), nbytes16, sink.data_ptr(), 512,
                                      torch.cuda.current_stream().cuda_stream)
        assert rc == 0
    rd_us = per_launch_us(torch, _R, _read, 4 * n_layer)
    res["read_floor_us"] = rd_us
    res["read_floor_GBps"] = kbytes / (rd_us * 1e-6) / 1e9
    res["kernel_frac_of_read_floor"] = rd_us / avg_us
    del rd
    if graph_ok and not args.no_graph:
        # The graph floor of the step's shape: two back-to-back launches per
        # layer of a one-thread kernel (an in-place add on one element), in a
        # graph of the same 2 x n_layer nodes. The step cannot go below it
        # with two launches per layer.
        one = torch.zeros(1, device="cuda")
        gf = make_graph(torch, b, lambda: [one.add_(1.0) for _ in range(2 * n_layer)])
        floor_s = time_region(torch, gf.replay, args.steps, args.warmup)
        res["launch_floor_us_per_layer"] = floor_s * 1e6 / n_layer
        res["us_per_layer"] = step_s * 1e6 / n_layer
        res["launch_floor_share"] = floor_s / step_s
    b.model.close()
    return res, step_bytes


def bench_prefill(torch, args, m, pos):
    n_layer = 2
    b = Bench(torch, n_layer, pos + m, m, seed=m + pos)
    b.fill_cache(pos + m, seed=3)
    flops = prefill_flops(m, pos)
    n = max(6, args.steps // 5)
    for i in range(3):
        b.model.dispatch_attention(b.a, b.q_off, b.out_off, i % n_layer, pos, m, True)
    torch.cuda.synchronize()
    avg_us = per_launch_us(
        torch, b, lambda i: b.model.dispatch_attention(b.a, b.q_off, b.out_off, i % n_layer, pos, m, True), n)
    tflops = flops / (avg_us * 1e-6) / 1e12
    # the chunk's two preceding dispatches: q norm + RoPE and the K/V writeback
    # (the q buffer is renormalized in place each call; the values stay finite)
    qn_us = per_launch_us(torch, b, lambda i: b.model.dispatch_q_norm_rope_fused(b.a, b.wp, b.q_off, 0, pos, m), n)
    wb_us = per_launch_us(torch, b, lambda i: b.model.dispatch_kv_writeback_fused(
        b.a, b.wp, b.k_off, b.v_off, b.cfg.head_dim, i % n_layer, pos, m), n)
    # The fused step (bp_dispatch_attention_prefill_step: q norm + RoPE, K/V
    # writeback and the attention kernel's f16 image in one preparation pass,
    # then the attention kernel), its preparation pass alone, and the three
    # separate dispatches it replaces.
    args_step = (b.a, b.wp, b.q_off, b.k_off, b.v_off, b.out_off, 0, b.cfg.head_dim)
    step_us = per_launch_us(torch, b, lambda i: b.model.dispatch_attention_prefill_step(
        *args_step, i % n_layer, pos, m), n)
    prep_us = per_launch_us(torch, b, lambda i: b.model.debug_prefill_prep(*args_step, i % n_layer, pos, m), n)

    def _unfused(i):
        b.model.dispatch_q_norm_rope_fused(b.a, b.wp, b.q_off, 0, pos, m)
        b.model.dispatch_kv_writeback_fused(b.a, b.wp, b.k_off, b.v_off, b.cfg.head_dim, i % n_layer, pos, m)
        b.model.dispatch_attention(b.a, b.q_off, b.out_off, i % n_layer, pos, m, True)
    unfused_us = per_launch_us(torch, b, _unfused, n)
    mfma_tf = bench_mfma_rate(torch, b) if m == 2048 and pos == 0 else None
    b.model.close()
    extra = {}
    if mfma_tf is not None:
        extra = {"mfma_sustained_random_TFLOPs": mfma_tf,
                 "frac_of_sustained_mfma": tflops / mfma_tf,
                 "step_attention_frac_of_sustained_mfma": flops / ((step_us - prep_us) * 1e-6) / 1e12 / mfma_tf}
    return {**extra, "m_tokens": m, "pos_base": pos, "flops": flops, "kernel_us_avg": avg_us,
            "TFLOPs": tflops, "frac_f16_mfma": tflops / F16_MFMA_PEAK_TFLOPS,
            "q_norm_rope_us": qn_us, "kv_writeback_us": wb_us,
            "kv_writeback_GBps": m * 8 * (2 * 256 + 2 * 144) / (wb_us * 1e-6) / 1e9,
            "step_us": step_us, "step_prep_us": prep_us, "step_unfused_us": unfused_us,
            "step_attention_us": step_us - prep_us,
            "step_attention_frac_f16_mfma": flops / ((step_us - prep_us) * 1e-6) / 1e12 / F16_MFMA_PEAK_TFLOPS}


def bench_mfma_rate(torch, b):
    """The f16 matrix rate this GPU sustains on real data (TFLOP/s): the bench
    library's bp_debug_mfma_rate (back-to-back v_mfma_f32_32x32x16_f16 on random
    f16 operands, one 4-wave workgroup per CU, 16384 x 4 MFMAs per wave) per
    launch in a graph after the warm-up. Random operands draw more power than
    constant ones, and the clock drops accordingly; this is the ceiling a
    prefill on real data can approach, beside the 2.5 PFLOP/s nominal peak
    that frac_f16_mfma is priced against."""
    from bonsai_pot_amd import lib as _lib
    n_wg = torch.cuda.get_device_properties(0).multi_processor_count
    iters = 16384
    sink = torch.zeros(n_wg * 256, device="cuda", dtype=torch.float32)

    class _R:
        model = b.model

    def _run(i):
        rc = _lib.bp_debug_mfma_rate(sink.data_ptr(), iters, n_wg, i + 1, torch.cuda.current_stream().cuda_stream)
        assert rc == 0
    us = per_launch_us(torch, _R, _run, 4)
    return n_wg * 4 * iters * 4 * 32768 / (us * 1e-6) / 1e12


def bench_copy(torch, args, nbytes=1 << 30):
    """Plain device-to-device copy of a known size: the calibration for HBM
    counters (FETCH_SIZE / WRITE_SIZE of this kernel vs nbytes read + written)
    and the achievable-bandwidth reference."""
    src = torch.ones(nbytes // 2, device="cuda", dtype=torch.float16)
    dst = torch.empty_like(src)
    for _ in range(3):
        dst.copy_(src)
    torch.cuda.synchronize()
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    n = max(5, args.steps // 5)
    start.record()
    for _ in range(n):
        dst.copy_(src)
    end.record()
    torch.cuda.synchronize()
    us = start.elapsed_time(end) * 1e3 / n
    return {"bytes_read": nbytes, "bytes_written": nbytes, "kernel_us_avg": us,
            "GBps_read_plus_write": 2 * nbytes / (us * 1e-6) / 1e9}


Q1_BYTES_PER_WEIGHT = 1 / 8 + 2 / 128     # Q1_0: 1 bit + one f16 scale per 128 weights


class MatvecLayers:
    """Bonsai-4B matvec weights of n_layer layers, each layer one byte buffer
    [qkv d | qkv qs | o d | o qs | gate/up d | gate/up qs | down d | down qs]
    (random signs, N(0, 0.02) f16 scales), plus an f16 activation buffer
    x [2560] | q [4096] | k [1024] | v [1024] | attn_out [4096] | gate [9728] |
    up [9728] | h [2560]."""
    HIDDEN, Q_DIM, KV_DIM, FFN = 2560, 4096, 1024, 9728

    def __init__(self, torch, n_layer, seed=0):
        from bonsai_pot_amd import Model, layout
        self.model = Model(layout.Config(n_layer=1), 64)
        self.model.set_stream(torch.cuda.current_stream().cuda_stream)
        g = torch.Generator(device="cuda").manual_seed(seed)
        H, Q, KV, F = self.HIDDEN, self.Q_DIM, self.KV_DIM, self.FFN
        self.tensors = {"qkv": (Q + 2 * KV, H), "o": (H, Q), "gate_up": (2 * F, H), "down": (H, F)}
        self.offs, at = {}, 0
        for name, (n, k) in self.tensors.items():
            nb = k // 128
            d_off = at
            qs_off = (d_off + 2 * n * nb + 255) // 256 * 256
            at = (qs_off + 16 * n * nb + 255) // 256 * 256
            self.offs[name] = (d_off, qs_off)
        self.layer_bytes = at
        self.bufs = []
        for _ in range(n_layer):
            buf = torch.randint(-128, 128, (at,), generator=g, device="cuda", dtype=torch.int8)
            for name, (n, k) in self.tensors.items():
                d_off, _ = self.offs[name]
                nd = n * (k // 128)
                d = (torch.randn(nd, generator=g, device="cuda") * 0.02).to(torch.float16)
                buf[d_off:d_off + 2 * nd].copy_(d.view(torch.int8))
            self.bufs.append(buf)
        self.x, self.q = 0, H
        self.k, self.v = H + Q, H + Q + KV
        self.attn, self.gate = H + Q + 2 * KV, H + 2 * Q + 2 * KV
        self.up, self.h = self.gate + F, self.gate + 2 * F
        self.act = torch.randn(self.h + H, generator=g, device="cuda").to(torch.float16)
        self.wn = (1 + 0.1 * torch.randn(2 * H, generator=g, device="cuda")).to(torch.float16)

    def weight_bytes(self, name):
        n, k = self.tensors[name]
        return int(n * k * Q1_BYTES_PER_WEIGHT)

    def launch(self, name, il):
        """One matvec of layer il, as the reference's decode layer issues it."""
        m, w, a, H = self.model, self.bufs[il].data_ptr(), self.act.data_ptr(), self.HIDDEN
        d_off, qs_off = self.offs[name]
        if name == "qkv":
            nb = H // 128
            Q, KV = self.Q_DIM, self.KV_DIM
            rng = [(d_off, qs_off, Q, self.q),
                   (d_off + 2 * Q * nb, qs_off + 16 * Q * nb, KV, self.k),
                   (d_off + 2 * (Q + KV) * nb, qs_off + 16 * (Q + KV) * nb, KV, self.v)]
            m.dispatch_matvec_q1_0_fused_normed(w, a, self.wn.data_ptr(), H, self.x, 0, rng)
        elif name == "o":
            m.dispatch_matvec_q1_0(w, a, self.Q_DIM, H, d_off, qs_off, self.attn, self.x, True)
        elif name == "gate_up":
            F, nb = self.FFN, H // 128
            rng = [(d_off, qs_off, F, self.gate), (d_off + 2 * F * nb, qs_off + 16 * F * nb, F, self.up)]
            m.dispatch_matvec_q1_0_fused_normed(w, a, self.wn.data_ptr(), H, self.x, H, rng)
        else:
            m.dispatch_matvec_q1_0_silu(w, a, self.FFN, H, d_off, qs_off, self.gate, self.up, self.x, True)


def bench_matvec(torch, args, n_layer=36):
    """The four Q1_0 matvec dispatches of a Bonsai-4B decode layer, over 36
    layers of distinct weights (520 MB, above the 256 MB Infinity Cache) so
    each launch streams its weights from HBM. Bytes = weights (1/8 + 2/128 B
    per weight) + f16 activations in and out."""
    b = MatvecLayers(torch, n_layer)
    names = list(b.tensors)
    for il in range(2):
        for nm in names:
            b.launch(nm, il)
    torch.cuda.synchronize()
    act_bytes = {"qkv": 2 * (2 * b.HIDDEN + 2 * b.HIDDEN) + 2 * 6144, "o": 2 * (b.Q_DIM + 2 * b.HIDDEN),
                 "gate_up": 2 * (2 * b.HIDDEN) + 2 * 2 * b.FFN, "down": 2 * (2 * b.FFN + 2 * b.HIDDEN)}
    res = {"layers": n_layer, "layer_weight_bytes": sum(b.weight_bytes(n) for n in names)}
    g = make_graph(torch, b, lambda: [b.launch(nm, il) for il in range(n_layer) for nm in names])
    step_s = time_region(torch, g.replay, max(5, args.steps // 5), 2)
    step_bytes = n_layer * sum(b.weight_bytes(n) + act_bytes[n] for n in names)
    res.update({"ms_per_step_36_layers": step_s * 1e3, "step_GBps": step_bytes / step_s / 1e9})
    for nm in names:
        us = per_launch_us(torch, b, lambda i, nm=nm: b.launch(nm, i % n_layer), n_layer)
        byt = b.weight_bytes(nm) + act_bytes[nm]
        res[nm] = {"n_k": b.tensors[nm], "kernel_us_avg": us, "bytes": byt,
                   "GBps": byt / (us * 1e-6) / 1e9, "frac_hbm": byt / (us * 1e-6) / 1e9 / HBM_PEAK_GBS}
    b.model.close()
    res["lm_head"] = bench_lm_head(torch, args)
    res["lm_head_mfma_opt_in"] = bench_lm_head(torch, args, arith="mfma")
    return res


def bench_lm_head(torch, args, vocab=151936, n_copies=8, arith=None):
    """The LM head matvec (vocab x 2560 Q1_0, 54.7 MB) over 8 copies of the
    weights (438 MB, above the Infinity Cache). arith None: the default
    arithmetic (the reference's f16 sums); "mfma": the opt-in i8-MFMA kernel."""
    from bonsai_pot_amd import Model, layout
    H = MatvecLayers.HIDDEN
    nb = H // 128
    old = os.environ.pop("BP_MATVEC_ARITH", None)
    if arith is not None:
        os.environ["BP_MATVEC_ARITH"] = arith
    try:
        m = Model(layout.Config(n_layer=1), 64)
    finally:
        os.environ.pop("BP_MATVEC_ARITH", None)
        if old is not None:
            os.environ["BP_MATVEC_ARITH"] = old
    m.set_stream(torch.cuda.current_stream().cuda_stream)
    g = torch.Generator(device="cuda").manual_seed(7)
    d_bytes = 2 * vocab * nb
    qs_off = (d_bytes + 255) // 256 * 256
    size = qs_off + 16 * vocab * nb
    bufs = []
    for _ in range(n_copies):
        buf = torch.randint(-128, 128, (size,), generator=g, device="cuda", dtype=torch.int8)
        d = (torch.randn(vocab * nb, generator=g, device="cuda") * 0.02).to(torch.float16)
        buf[:d_bytes].copy_(d.view(torch.int8))
        bufs.append(buf)
    act = torch.randn(H + vocab, generator=g, device="cuda").to(torch.float16)

    class _B:
        model = m
    launch = lambda i: m.dispatch_matvec_q1_0(bufs[i % n_copies].data_ptr(), act.data_ptr(), H, vocab, 0, qs_off,
                                              0, H, False)
    for i in range(n_copies):
        launch(i)
    torch.cuda.synchronize()
    us = per_launch_us(torch, _B, launch, 2 * n_copies)
    byt = int(vocab * H * Q1_BYTES_PER_WEIGHT) + 2 * (H + vocab)
    # top-k (k = 32) of the head's logits, as the step's last dispatch
    res = torch.zeros(64, dtype=torch.int32, device="cuda")
    topk = lambda i: m.dispatch_topk_reduce(act.data_ptr(), res.data_ptr(), vocab, 32, H, 0)
    topk(0)
    torch.cuda.synchronize()
    tk_us = per_launch_us(torch, _B, topk, 8)
    m.close()
    return {"n_k": [vocab, H], "kernel_us_avg": us, "bytes": byt, "GBps": byt / (us * 1e-6) / 1e9,
            "frac_hbm": byt / (us * 1e-6) / 1e9 / HBM_PEAK_GBS,
            "topk_reduce_k32": {"n": vocab, "us_avg": tk_us, "bytes": 2 * vocab,
                                "note": "one 1024-thread workgroup, latency-bound"}}


def bench_matmul(torch, args, m_tokens=512, n_layer=8):
    """The Bonsai-4B prefill projections of one layer at m_tokens tokens:
    quantize_act (Q8_0) of each input, then the Q1_0 x Q8_0 matmul (q/k/v
    6144x2560, o 2560x4096, gate/up 19456x2560, down 2560x9728), over n_layer
    layers of distinct weights. Work = 2 m n k integer ops per matmul
    (i8 MFMA peak 5.0 POP/s)."""
    b = MatvecLayers(torch, n_layer, seed=3)
    m = b.model
    g = torch.Generator(device="cuda").manual_seed(11)
    kmax = max(k for _, k in b.tensors.values())
    nmax = max(n for n, _ in b.tensors.values())
    x = torch.randn(m_tokens * kmax, generator=g, device="cuda").to(torch.float16)
    y = torch.zeros(m_tokens * nmax, device="cuda", dtype=torch.float16)
    q8 = torch.empty(m_tokens * kmax + m_tokens * kmax // 8, device="cuda", dtype=torch.int8)
    qs_off = m_tokens * kmax // 8

    def quant(name):
        _, k = b.tensors[name]
        m.dispatch_quantize_act(x.data_ptr(), q8.data_ptr(), k, m_tokens, 0, 0, qs_off)

    def mm(name, il):
        n, k = b.tensors[name]
        d_off, w_qs = b.offs[name]
        m.dispatch_matmul_q1_0(b.bufs[il].data_ptr(), q8.data_ptr(), y.data_ptr(), k, n, m_tokens,
                               d_off, w_qs, 0, qs_off, 0, name in ("o", "down"))

    res = {"m_tokens": m_tokens, "layers": n_layer}
    total_us, total_ops = 0.0, 0
    for nm, (n, k) in b.tensors.items():
        quant(nm)
        mm(nm, 0)
        torch.cuda.synchronize()
        us = per_launch_us(torch, b, lambda i, nm=nm: mm(nm, i % n_layer), n_layer)
        q_us = per_launch_us(torch, b, lambda i, nm=nm: quant(nm), 4)
        ops = 2 * m_tokens * n * k
        total_us += us + q_us
        total_ops += ops
        res[nm] = {"n_k": [n, k], "matmul_us_avg": us, "quantize_us_avg": q_us, "ops": ops,
                   "TOPS": ops / (us * 1e-6) / 1e12, "frac_i8_mfma": ops / (us * 1e-6) / 1e12 / I8_MFMA_PEAK_TOPS}
    res["layer_us"] = total_us
    res["layer_TOPS"] = total_ops / (total_us * 1e-6) / 1e12
    m.close()
    return res


def measured_traffic(workload, kernel):
    """HBM bytes per dispatch of `kernel` in `workload`, measured with rocprofv3
    FETCH_SIZE / WRITE_SIZE (scaled by a copy kernel of known size), from
    profiles/traffic.json (keys "workload:kernel:grid")."""
    path = os.path.join(ROOT, "profiles", "traffic.json")
    if not os.path.exists(path):
        return None
    with open(path) as f:
        table = json.load(f)["bytes_per_dispatch"]
    hits = [v for k, v in table.items() if k.startswith(f"{workload}:{kernel}:")]
    return hits[0] if len(hits) == 1 else None


def _cpu_info():
    """CPU model of the host and its physical core count. The model name from
    /proc/cpuinfo (a virtual machine may report only the vendor's family
    name there), completed with the CPU family / model / stepping numbers and
    lscpu's BIOS model name where they are available."""
    import subprocess
    name, cores, ids = "unknown", set(), {}
    try:
        phys = core = None
        with open("/proc/cpuinfo") as f:
            for line in f:
                k, _, v = line.partition(":")
                k, v = k.strip(), v.strip()
                if k == "model name" and name == "unknown":
                    name = v
                elif k in ("cpu family", "model", "stepping") and k not in ids:
                    ids[k] = v
                elif k == "physical id":
                    phys = v
                elif k == "core id":
                    core = v
                elif not k and phys is not None:
                    cores.add((phys, core))
                    phys = core = None
        if phys is not None:
            cores.add((phys, core))
    except OSError:
        pass
    extra = []
    if ids:
        extra.append(", ".join(f"{k} {v}" for k, v in ids.items()))
    try:
        out = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=10).stdout
        for line in out.splitlines():
            k, _, v = line.partition(":")
            if k.strip() == "BIOS Model name" and v.strip() and v.strip() != name:
                extra.append("BIOS model name " + v.strip())
    except (OSError, subprocess.SubprocessError):
        pass
    if extra:
        name = f"{name} ({'; '.join(extra)})"
    return name, len(cores) or None


def cpu_baseline(seconds=10.0):
    """CPU oracle (plain-C restatement of the reference's split/merge decode)
    on the host: decode at ctx 4096, one layer-decode per call, run by a pool
    of threads (the C calls release the GIL), each on its own output buffer,
    for ~seconds. Threads = this process's CPU share, capped at 16 (the GPU
    box grants 16 host CPUs to a one-GPU job)."""
    import numpy as np
    from concurrent.futures import ThreadPoolExecutor
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle as orc
    from bonsai_pot_amd import layout
    n_keys, max_seq, n_layer = 4097, 4097, 4
    nbytes = layout.kv_buffer_bytes(n_layer, 1024, max_seq)
    rng = np.random.default_rng(0)
    kv = []
    for _ in range(2):
        buf = rng.integers(-127, 128, nbytes, dtype=np.int8).view(np.uint8)
        nd = n_layer * max_seq * 32
        buf[:nd * 4].view(np.float32)[:] = np.float32(0.02)
        kv.append(buf)
    act0 = rng.standard_normal(2 * 4096).astype(np.float16).view(np.uint16)
    try:
        share = len(os.sched_getaffinity(0))
    except AttributeError:
        share = os.cpu_count() or 1
    threads = max(1, min(share, int(os.environ.get("OMP_NUM_THREADS", "16") or 16), 16))
    params = []
    for il in range(n_layer):
        d_word, qs_byte = layout.kv_layer_offsets(n_layer, 1024, max_seq, il)
        params.append(orc.AttnSplitParams(head_dim=128, n_head=32, n_kv_head=8, pos=n_keys, kv_stride=1024,
                                          q_offset=0, k_d_word_offset=d_word, k_qs_byte_offset=qs_byte,
                                          v_d_word_offset=d_word, v_qs_byte_offset=qs_byte,
                                          n_chunks_active=(n_keys + 15) // 16, scale=128 ** -0.5,
                                          out_offset=4096))
    t_end = [0.0]

    def worker(tid):
        act = act0.copy()
        done = 0
        while time.perf_counter() < t_end[0]:
            orc.attention_split_merge(params[(tid + done) % n_layer], act, kv[0], kv[1])
            done += 1
        return done

    t0 = time.perf_counter()
    t_end[0] = t0 + seconds
    with ThreadPoolExecutor(max_workers=threads) as ex:
        layers = sum(ex.map(worker, range(threads)))
    dt = time.perf_counter() - t0
    name, phys = _cpu_info()
    return {"value": decode_bytes(n_keys) * layers / dt / 1e9, "unit": "GB/s", "cores": threads,
            "kind": "port", "cpu": name, "cpu_physical_cores_on_host": phys, "cpu_share": share,
            "sample": f"{layers} layer-decodes at ctx 4096 (4097 rows, 32 q heads) in {dt:.1f} s on "
                      f"{threads} threads, plain-C oracle restating attention_split + attention_merge "
                      "(the reference's WGSL on lavapipe cannot run here: no Vulkan loader/ICD, no Rust)"}


def roofline_decode(d4):
    """Dominant kernel pair of the headline step: decode_split_kernel<true, 1> +
    decode_merge_kernel<true, 8>, i.e. one layer of the fused decode step.
    achieved = algorithmic bytes of one layer (4097 rows x 2304 B + q in/out)
    / the per-layer time of the timed region (HIP events, graph replays)."""
    per_layer_s = d4["ms_per_step"] * 1e-3 / d4["layers"]
    achieved = d4["kernel_bytes"] / per_layer_s / 1e9
    split = measured_traffic("decode4k", "decode_split_kernel<true, 1>")
    merge = measured_traffic("decode4k", "decode_merge_kernel<true, 8>")
    traffic = None if split is None or merge is None else split + merge
    return {"bound": "hbm", "achieved": achieved, "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": achieved / HBM_PEAK_GBS, "traffic": traffic,
            "kernel": "decode_split_kernel<true, 1> + decode_merge_kernel<true, 8> (one layer of the fused step)",
            "bytes_per_launch": d4["kernel_bytes"], "us_per_launch": per_layer_s * 1e6}


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py runs on one GPU only: --gpus {args.gpus} is not supported (this build "
              "measures one MI355X; multi-GPU sharding is design-only)", file=sys.stderr)
        sys.exit(2)
    import torch
    assert torch.cuda.is_available(), "bench.py needs a HIP device"
    torch.cuda.init()
    extras = {}
    if args.only in (None, "decode4k"):
        d4, step_bytes = bench_decode(torch, args, 4096, 36)
        extras["decode_ctx4096_36layers"] = d4
    if args.only in (None, "decode32k"):
        d32, _ = bench_decode(torch, args, 32768, 8)
        extras["decode_ctx32768"] = d32
    if args.only in (None, "prefill"):
        extras["prefill_pp2048"] = bench_prefill(torch, args, 2048, 0)
        extras["prefill_pp512"] = bench_prefill(torch, args, 512, 0)
    if args.only in (None, "chunked"):
        extras["chunked_prefill_2048_on_2048"] = bench_prefill(torch, args, 2048, 2048)
        # a short chunk over a long cache (a chat turn): the key-split layout
        extras["chunked_prefill_64_on_16384"] = bench_prefill(torch, args, 64, 16384)
    if args.only in (None, "matvec"):
        extras["matvec_q1_0_4b_layer"] = bench_matvec(torch, args)
    if args.only in (None, "matmul"):
        extras["matmul_q1_0_q8_0_4b_layer_pp512"] = bench_matmul(torch, args)
    if args.only == "copy":
        extras["copy_1GiB"] = bench_copy(torch, args)
    if args.only is not None:
        print(json.dumps(extras), flush=True)
        return
    cpu = None if args.skip_cpu else cpu_baseline()
    out = {
        "metric": METRIC,
        "value": d4["step_GBps"],
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": d4["ms_per_step"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32 (i8 Q8_0 cache, f16 q/out)",
        "data": "synthetic (seeded N(0,1) q/k/v through kv_writeback; no model weights)",
        "config": {"workload": "configs[1]: Bonsai-4B decode attention, 36 layers, ctx 4096, batch 1 "
                               "(fused q_norm_rope + kv_writeback + split-K decode per layer, HIP graph)",
                   "n_head": 32, "n_kv_head": 8, "head_dim": 128, "ctx": 4096, "layers": 36,
                   "parallelism": "none (1 GPU)"},
        "roofline": roofline_decode(d4),
        "cpu_baseline": cpu,
        **extras,
    }
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
