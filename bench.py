#!/usr/bin/env python3
"""Benchmark of the MI355X quantized-matmul hot path (one GPU).

Headline: Q4_K decode GEMV, weight 14336x4096,
f32 activation of 4096, one launch per step over a weight copy rotated among
16 device copies (528 MB > the 256 MB Infinity Cache) so bytes come from HBM.
value = algorithmic bytes per launch / mean launch time over K timed launches
(HIP events on the launch stream).

The same JSON line carries the other configs as `extra`: Q8_0 and Q6_K GEMV
(configs 0, 2), the Q4_K prefill GEMM at M=512 (config 3) and the LLaMA-8B
shape greedy decode (config 4), the Q5_K GEMV and the headline shape on the
int8 dot-product path, the Q6_K and Q8_0 GEMMs at M=512 and the 8B shape with the
Q4_K_M format mix (and, on request, GGUF-order F16 / Q2_K GEMVs), plus
`roofline` for the headline kernel and
`cpu_baseline`: the oracle's restatement of the reference's AVX2 path on one
host core over a bounded sample of the same workload (and, in `extra`, the
reference's scalar kernel with its output rows spread over up to 16 host
threads, as its rayon callers spread them).
"""
import argparse
import ctypes
import json
import os
import platform
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
INT8_PEAK_TOPS = 5000.0
FP16_PEAK_TFLOPS = 2500.0


def algorithmic_bytes(dtype, n, k):
    be, bb = {1: (1, 2), 8: (32, 34), 10: (256, 84), 11: (256, 110), 12: (256, 144), 13: (256, 176),
              14: (256, 210)}[dtype]
    return n * (k // be) * bb + k * 4 + n * 4


def make_weights(torch, A, dtype, n, k, copies, seed):
    L = A.lib()
    be, bb = A.block_geometry(dtype)
    nblk = n * (k // be)
    ws = []
    raws = []
    for i in range(copies):
        raw = torch.empty(nblk * bb, dtype=torch.uint8, device="cuda")
        A.check(L.aeth_fill_synthetic_raw(dtype, seed + i, raw.data_ptr(), nblk, None), "fill")
        w = ctypes.c_void_p()
        A.check(L.aeth_weight_create(dtype, n, k, raw.data_ptr(), 1, None, ctypes.byref(w)), "weight_create")
        ws.append(w)
        if i == 0:
            raws.append(raw)
        else:
            del raw
    torch.cuda.synchronize()
    return ws, raws


def time_launches(torch, fn, steps, warmup):
    """Mean ms per launch of `steps` back-to-back launches on the current stream,
    bracketed by HIP events on that stream. A bounded spin kernel (torch's
    clock-based _sleep, ~5 ms) is queued first so that every timed launch is
    already enqueued when the start event fires: the figure is the GPU's, not
    the rate at which Python can enqueue."""
    stream = torch.cuda.current_stream()
    for i in range(warmup):
        fn(i)
    torch.cuda.synchronize()
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    torch.cuda._sleep(int(2.4e9 * max(0.005, steps * 30e-6)))
    e0.record(stream)
    for i in range(steps):
        fn(i)
    e1.record(stream)
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / steps  # ms per launch


def bench_gemv(torch, A, dtype, n, k, steps, warmup, copies=16, seed=0xAE7E40, flags=0):
    L = A.lib()
    ws, raws = make_weights(torch, A, dtype, n, k, copies, seed)
    x = torch.empty(k, dtype=torch.float32, device="cuda")
    A.check(L.aeth_fill_normal_f32(seed ^ 0x55, x.data_ptr(), k, 0.0, 1.0, None))
    y = torch.empty(n, dtype=torch.float32, device="cuda")
    s = torch.cuda.current_stream().cuda_stream

    def step(i):
        rc = L.aeth_qmatmul(ws[i % copies], x.data_ptr(), 1, y.data_ptr(), flags, s)
        if rc:
            A.check(rc, "qmatmul")

    ms = time_launches(torch, step, steps, warmup)
    for w in ws:
        L.aeth_weight_free(w)
    nbytes = algorithmic_bytes(dtype, n, k)
    return {"ms": ms, "gbs": nbytes / (ms * 1e-3) / 1e9, "bytes": nbytes, "raw0": raws[0], "x": x}


def bench_read_floor(torch, A, nbytes, steps, warmup, copies=16):
    """The plain streaming read (aeth_stream_read) of nbytes, rotated over as
    many device buffers as the GEMV's weight copies: what one launch of that
    size can stream from HBM on this box."""
    L = A.lib()
    bufs = [torch.ones(nbytes, dtype=torch.uint8, device="cuda") for _ in range(copies)]
    sink = torch.zeros(1 << 20, dtype=torch.int32, device="cuda")
    s = torch.cuda.current_stream().cuda_stream

    def step(i):
        A.check(L.aeth_stream_read(bufs[i % copies].data_ptr(), nbytes, sink.data_ptr(), sink.numel(), s), "read")

    ms = time_launches(torch, step, steps, warmup)
    del bufs
    return {"ms": ms, "gbs": nbytes / (ms * 1e-3) / 1e9}


def bench_mfma_rate(torch, A, kind, iters=2000, workgroups=256):
    """Matrix-core rate the box sustains (aeth_mfma_rate): kind 0 fp16
    v_mfma_f32_32x32x16_f16, kind 1 int8 v_mfma_i32_32x32x32_i8, one wave per
    SIMD of independent MFMAs on register operands; TFLOP/s or TOP/s."""
    L = A.lib()
    sink = torch.empty(workgroups * 256, dtype=torch.float32, device="cuda")
    s = torch.cuda.current_stream().cuda_stream

    def step(i):
        A.check(L.aeth_mfma_rate(kind, iters, workgroups, sink.data_ptr(), s), "mfma_rate")

    ms = time_launches(torch, step, 5, 2)
    ops = (32768 if kind == 0 else 65536) * 8 * iters * workgroups * 4
    return ops / (ms * 1e-3) / 1e12


def bench_gemm(torch, A, n, k, m, steps, warmup, seed=0xAE7E43, flags=0):
    L = A.lib()
    copies = 2
    ws, raws = make_weights(torch, A, 12, n, k, copies, seed)
    a = torch.empty(m * k, dtype=torch.float32, device="cuda")
    A.check(L.aeth_fill_normal_f32(seed ^ 0x77, a.data_ptr(), m * k, 0.0, 1.0, None))
    c = torch.empty(m * n, dtype=torch.float32, device="cuda")
    s = torch.cuda.current_stream().cuda_stream

    def step(i):
        A.check(L.aeth_qmatmul(ws[i % copies], a.data_ptr(), m, c.data_ptr(), flags, s), "gemm")

    ms = time_launches(torch, step, steps, warmup)
    for w in ws:
        L.aeth_weight_free(w)
    return {"ms": ms, "tflops": 2.0 * m * n * k / (ms * 1e-3) / 1e12, "raw0": raws[0], "a": a}


def bench_batched(torch, A, dtype, n, k, m, steps, warmup, seed=0xAE7E47):
    L = A.lib()
    ws, _ = make_weights(torch, A, dtype, n, k, 2, seed)
    a = torch.empty(m * k, dtype=torch.float32, device="cuda")
    A.check(L.aeth_fill_normal_f32(seed ^ 0x77, a.data_ptr(), m * k, 0.0, 1.0, None))
    c = torch.empty(m * n, dtype=torch.float32, device="cuda")
    s = torch.cuda.current_stream().cuda_stream

    def step(i):
        A.check(L.aeth_qmatmul(ws[i % 2], a.data_ptr(), m, c.data_ptr(), 0, s), "batched")

    ms = time_launches(torch, step, steps, warmup)
    for w in ws:
        L.aeth_weight_free(w)
    return {"ms": ms, "tflops": 2.0 * m * n * k / (ms * 1e-3) / 1e12}


def bench_decode(torch, A, n_tokens=128, prefilled=2048, prefill_tokens=512, want_cpu=False):
    L = A.lib()
    cfg = A.LlamaConfig(vocab_size=128256, d_model=4096, num_layers=32, num_heads=32, num_kv_heads=8, head_dim=128,
                        d_ff=14336, max_seq_len=4096, rope_base=500000.0, rms_norm_eps=1e-5)
    dt = (ctypes.c_int32 * (32 * 7))(*([12] * (32 * 7)))
    r = ctypes.c_void_p()
    t0 = time.time()
    A.check(L.aeth_runner_create(ctypes.byref(cfg), None, dt, None, None, None, 14, None, 0x8B8B8B,
                                 ctypes.byref(r)), "runner_create")
    setup_s = time.time() - t0
    toks = (ctypes.c_int32 * n_tokens)()
    A.check(L.aeth_runner_fill_kv(r, 0x4B56, prefilled), "fill_kv")
    A.check(L.aeth_runner_generate(r, 1, prefilled, 2, toks, 1), "warmup generate")
    A.check(L.aeth_runner_fill_kv(r, 0x4B56, prefilled), "fill_kv")
    t0 = time.perf_counter()
    A.check(L.aeth_runner_generate(r, 1, prefilled, n_tokens, toks, 1), "generate")
    dt_s = time.perf_counter() - t0
    # batched prefill of a 512-token prompt (forward_batch): one warm-up, then timed
    prompt = (ctypes.c_int32 * prefill_tokens)(*[(7919 * i + 13) % 128256 for i in range(prefill_tokens)])
    A.check(L.aeth_runner_prefill(r, prompt, prefill_tokens, None, None), "prefill warmup")
    reps = 3
    t0 = time.perf_counter()
    for _ in range(reps):
        A.check(L.aeth_runner_prefill(r, prompt, prefill_tokens, None, None), "prefill")
    pf_s = (time.perf_counter() - t0) / reps
    # a short prompt: 32 tokens, where the GEMMs' tiles are fewer than the CUs (K split over workgroups)
    short = (ctypes.c_int32 * 32)(*[(7919 * i + 13) % 128256 for i in range(32)])
    A.check(L.aeth_runner_prefill(r, short, 32, None, None), "short prefill warmup")
    t0 = time.perf_counter()
    for _ in range(reps):
        A.check(L.aeth_runner_prefill(r, short, 32, None, None), "short prefill")
    pf32_s = (time.perf_counter() - t0) / reps
    cpu_model = export_decode_model(A, r, cfg, prefilled, [1] + list(toks)[:7]) if want_cpu else None
    L.aeth_runner_free(r)
    layer_weights = 4096 * 4096 * 2 + 1024 * 4096 * 2 + 14336 * 4096 * 3
    pf_flops = 2.0 * prefill_tokens * 32 * layer_weights + 2.0 * 128256 * 4096
    # weight bytes + f32 KV read (avg over steps) + KV write, per step
    q4 = 32 * (4096 * 16 * 144 * 2 + 1024 * 16 * 144 * 2 + 14336 * 16 * 144 * 2 + 4096 * 56 * 144)
    q6 = 128256 * 16 * 210
    kv_avg = 32 * 2 * 8 * 128 * 4 * (prefilled + 1 + (n_tokens - 1) / 2.0)
    step_bytes = q4 + q6 + kv_avg + (32 * 2 + 1) * 4096 * 4
    return {"tok_s": n_tokens / dt_s, "ms_per_token": dt_s * 1e3 / n_tokens, "setup_s": setup_s,
            "gbs": step_bytes * n_tokens / dt_s / 1e9, "step_bytes": step_bytes, "first_tokens": list(toks)[:8],
            "prefill_tok_s": prefill_tokens / pf_s, "prefill_ms": pf_s * 1e3, "prefill_tflops": pf_flops / pf_s / 1e12,
            "prefill32_ms": pf32_s * 1e3,
            "cpu_model": cpu_model}


def bench_q4_k_m(torch, A, n_tokens=64, prefilled=2048, prefill_tokens=512, layer_dtypes=(12, 12, 14, 12, 12, 12, 14),
                 mix="Q4_K_M: attn_v, ffn_down Q6_K; q, k, o, gate, up Q4_K; LM head Q6_K"):
    """bench_decode's model with llama.cpp's Q4_K_M mix: attn_v and ffn_down in Q6_K, the
    other five layer weights Q4_K (q|k one weight, v another; in prefill the Q6_K projections
    take the Q6_K GEMM), or another per-layer mix (`layer_dtypes`: q k v o gate up down)."""
    L = A.lib()
    cfg = A.LlamaConfig(vocab_size=128256, d_model=4096, num_layers=32, num_heads=32, num_kv_heads=8, head_dim=128,
                        d_ff=14336, max_seq_len=4096, rope_base=500000.0, rms_norm_eps=1e-5)
    dt = (ctypes.c_int32 * (32 * 7))(*(list(layer_dtypes) * 32))
    r = ctypes.c_void_p()
    A.check(L.aeth_runner_create(ctypes.byref(cfg), None, dt, None, None, None, 14, None, 0x8B8B8B,
                                 ctypes.byref(r)), "runner_create")
    toks = (ctypes.c_int32 * n_tokens)()
    A.check(L.aeth_runner_fill_kv(r, 0x4B56, prefilled), "fill_kv")
    A.check(L.aeth_runner_generate(r, 1, prefilled, 2, toks, 1), "warmup generate")
    A.check(L.aeth_runner_fill_kv(r, 0x4B56, prefilled), "fill_kv")
    t0 = time.perf_counter()
    A.check(L.aeth_runner_generate(r, 1, prefilled, n_tokens, toks, 1), "generate")
    dt_s = time.perf_counter() - t0
    prompt = (ctypes.c_int32 * prefill_tokens)(*[(7919 * i + 13) % 128256 for i in range(prefill_tokens)])
    A.check(L.aeth_runner_prefill(r, prompt, prefill_tokens, None, None), "prefill warmup")
    reps = 3
    t0 = time.perf_counter()
    for _ in range(reps):
        A.check(L.aeth_runner_prefill(r, prompt, prefill_tokens, None, None), "prefill")
    pf_s = (time.perf_counter() - t0) / reps
    L.aeth_runner_free(r)
    layer_weights = 4096 * 4096 * 2 + 1024 * 4096 * 2 + 14336 * 4096 * 3
    pf_flops = 2.0 * prefill_tokens * 32 * layer_weights + 2.0 * 128256 * 4096
    return {"decode_tok_s": round(n_tokens / dt_s, 1), "ms_per_token": round(dt_s * 1e3 / n_tokens, 4),
            "prefill_tok_s": round(prefill_tokens / pf_s, 1), "prefill_ms": round(pf_s * 1e3, 3),
            "prefill_TFLOP/s": round(pf_flops / pf_s / 1e12, 1), "prefill_tokens": prefill_tokens,
            "decode_tokens": n_tokens, "prefilled": prefilled, "mix": mix}


def bench_decode_eager(torch, A, n_tokens=128, prefilled=2048):
    """The decode step of bench_decode's model without the HIP graph: each token's
    kernels are launched one by one (aeth_runner_generate with use_graph = 0).
    Not in the default sections; its launches carry no graph, so per-dispatch
    counters (rocprofv3 --pmc) can be collected over it."""
    L = A.lib()
    cfg = A.LlamaConfig(vocab_size=128256, d_model=4096, num_layers=32, num_heads=32, num_kv_heads=8, head_dim=128,
                        d_ff=14336, max_seq_len=4096, rope_base=500000.0, rms_norm_eps=1e-5)
    dt = (ctypes.c_int32 * (32 * 7))(*([12] * (32 * 7)))
    r = ctypes.c_void_p()
    A.check(L.aeth_runner_create(ctypes.byref(cfg), None, dt, None, None, None, 14, None, 0x8B8B8B,
                                 ctypes.byref(r)), "runner_create")
    toks = (ctypes.c_int32 * n_tokens)()
    A.check(L.aeth_runner_fill_kv(r, 0x4B56, prefilled), "fill_kv")
    A.check(L.aeth_runner_generate(r, 1, prefilled, 2, toks, 0), "warmup generate")
    A.check(L.aeth_runner_fill_kv(r, 0x4B56, prefilled), "fill_kv")
    t0 = time.perf_counter()
    A.check(L.aeth_runner_generate(r, 1, prefilled, n_tokens, toks, 0), "generate (eager)")
    dt_s = time.perf_counter() - t0
    L.aeth_runner_free(r)
    return {"tok_s": n_tokens / dt_s, "ms_per_token": dt_s * 1e3 / n_tokens, "tokens": n_tokens,
            "first_tokens": list(toks)[:8]}


def export_decode_model(A, r, cfg, prefilled, tokens):
    """Host copies of what the CPU decode step reads: every layer weight (raw
    GGUF row blocks), the norms, the LM head, the KV cache refilled to
    `prefilled` positions, and the embedding rows of `tokens` (the GPU's greedy
    tokens, so both sides decode the same sequence)."""
    import numpy as np

    L = A.lib()

    def ex(which, l, nbytes, dt=np.uint8):
        buf = np.empty(nbytes // np.dtype(dt).itemsize, dtype=dt)
        A.check(L.aeth_runner_export(r, which, l, buf.ctypes.data, nbytes), "export")
        return buf

    d, dff, kvd, nl = cfg.d_model, cfg.d_ff, cfg.num_kv_heads * cfg.head_dim, cfg.num_layers
    rowb = lambda k: (k // 256) * 144
    sizes = [d * rowb(d), kvd * rowb(d), kvd * rowb(d), d * rowb(d), dff * rowb(d), dff * rowb(d), d * rowb(dff)]
    A.check(L.aeth_runner_fill_kv(r, 0x4B56, prefilled), "fill_kv")
    kv = np.empty((nl, 2, cfg.num_kv_heads, cfg.max_seq_len, cfg.head_dim), np.float32)
    fill = ctypes.c_int32()
    A.check(L.aeth_runner_kv_to_host(r, kv.ctypes.data, ctypes.byref(fill)), "kv_to_host")
    return {"cfg": cfg, "layers": [[ex(j, l, sizes[j]) for j in range(7)] for l in range(nl)],
            "norms": [[ex(7 + j, l, d * 4, np.float32) for j in range(2)] for l in range(nl)],
            "final": ex(9, 0, d * 4, np.float32), "lm": ex(10, 0, cfg.vocab_size * 16 * 210), "kv": kv,
            "prefilled": prefilled, "tokens": tokens, "emb": [ex(11, t, d * 4, np.float32) for t in tokens]}


def profile_traffic(name):
    """HBM bytes per dispatch recorded in profiles/<name>_traffic.json, or None."""
    try:
        with open(os.path.join(ROOT, "profiles", name + "_traffic.json")) as f:
            return json.load(f)["traffic_bytes_per_dispatch"]
    except (OSError, ValueError, KeyError):
        return None


def measured_traffic():
    """HBM bytes per headline GEMV dispatch from the committed rocprofv3 PMC
    summary (FETCH_SIZE + WRITE_SIZE, calibrated on a copy of known size)."""
    p = os.path.join(ROOT, "profiles", "q4k_gemv_14336x4096_traffic.json")
    try:
        with open(p) as f:
            return json.load(f)["traffic_bytes_per_dispatch"]
    except (OSError, ValueError, KeyError):
        return None


def cpu_rows_parallel(raw, x, n, k, seconds=4.0):
    """Secondary CPU figure: the reference's scalar Q4_K kernel (q4_k.rs, whose
    callers spread output rows over cores with rayon) restated in oracle/oracle.c,
    its output rows split evenly across up to 16 host threads (ctypes releases
    the GIL during each call)."""
    import concurrent.futures
    from oracle import oracle as O

    threads = max(1, min(16, len(os.sched_getaffinity(0))))
    row_bytes = (k // 256) * 144
    parts = [(n * t // threads, n * (t + 1) // threads) for t in range(threads)]

    def run(pr):
        r0, r1 = pr
        O.scalar_matmul(12, x, raw[r0 * row_bytes:r1 * row_bytes], 1, r1 - r0, k)

    calls = 0
    with concurrent.futures.ThreadPoolExecutor(threads) as ex:
        t0 = time.perf_counter()
        while True:
            list(ex.map(run, parts))
            calls += 1
            el = time.perf_counter() - t0
            if el >= seconds:
                break
    nbytes = algorithmic_bytes(12, n, k)
    return {"value": round(nbytes * calls / el / 1e9, 3), "unit": "GB/s", "cores": threads,
            "kind": "port (scalar kernel, rows over threads)", "cpu": cpu_name(), "nproc": os.cpu_count(),
            "sample": "%d full Q4_K GEMVs 14336x4096 in %.1f s" % (calls, el)}


def bench_boundary(torch, A, dtype, n, k, raw_dev, device_us, calls=20):
    """The plugin boundary (QuantKernel::matmul, registry.rs:7-19, reached from
    quantized_matmul_impl, dispatch.rs:120): aeth_quantized_matmul_impl on host
    slices — a f32[k] and c f32[n] in pageable host memory, the weight bytes in
    host memory and already in the library's device cache (one warm-up call
    uploads them). Per call: the content fingerprint of the whole weight (the
    cache's check that the slice was not rewritten), the copy of a to the
    device, the GEMV, the copy of c back and the stream synchronisation.
    Wall-clock median over `calls` calls; the fingerprint is also timed alone."""
    import numpy as np

    L = A.lib()
    raw = raw_dev.cpu().numpy()
    a = np.random.default_rng(5).standard_normal(k).astype(np.float32)
    c = np.empty(n, np.float32)

    def call():
        A.check(L.aeth_quantized_matmul_impl(a.ctypes.data, 1, raw.ctypes.data, raw.nbytes, n, k, dtype,
                                             c.ctypes.data), "quantized_matmul_impl")

    call()  # uploads the weight into the cache
    med, _ = cpu_median(call, calls)
    fpv = ctypes.c_uint64()
    fmed, _ = cpu_median(lambda: A.check(L.aeth_weight_fingerprint(raw.ctypes.data, raw.nbytes, ctypes.byref(fpv))),
                         calls)
    return {"us_per_call": round(med * 1e6, 1), "device_gemv_us": round(device_us, 3),
            "fingerprint_us": round(fmed * 1e6, 1), "fingerprint_GB/s": round(raw.nbytes / fmed / 1e9, 2),
            "weight_bytes": int(raw.nbytes), "copies_bytes": int(4 * (k + n)),
            "host_threads": min(8, os.cpu_count() or 1),
            "note": "median wall-clock of %d host-slice calls, weight cached on the device; "
                    "fingerprint = hash of every weight byte per call" % calls}


def cpu_name():
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor() or platform.machine()


def cpu_median(fn, runs):
    ts = []
    for _ in range(runs):
        t0 = time.perf_counter()
        fn()
        ts.append(time.perf_counter() - t0)
    ts.sort()
    return ts[len(ts) // 2], ts


def cpu_configs(q8, q6, gemm, dec):
    """CPU figures beside the other configs, on one pinned core (the reference's
    AVX2 kernels are single-threaded): C1 the scalar Q8_0 kernel q8_0.rs (the
    reference's AVX2 Q8_0 kernel mis-addresses its quants, avx2.rs:163), median
    of 5; C3 avx2::matmul_q6_k, median of 5; C4 one m = 512 avx2::matmul_q4_k
    call per N; C5 the CPU decode step (forward_one_internal's CPU branch,
    runner.rs:1557-1646) per token over 8 steps of the GPU's greedy sequence."""
    from oracle import oracle as O

    out = {}
    host = cpu_name()
    if q8 is not None:
        raw, x = q8
        med, ts = cpu_median(lambda: O.scalar_matmul(8, x, raw, 1, 4096, 4096), 5)
        out["q8_0_gemv_4096x4096"] = {"value": round(algorithmic_bytes(8, 4096, 4096) / med / 1e9, 3), "unit": "GB/s",
                                      "cores": 1, "kind": "port", "cpu": host, "nproc": os.cpu_count(),
                                      "sample": "median of 5 full GEMVs (scalar q8_0.rs restated): %.2f ms" % (med * 1e3)}
        print("[bench] cpu C1: %s" % out["q8_0_gemv_4096x4096"], file=sys.stderr, flush=True)
    if q6 is not None:
        raw, x = q6
        med, ts = cpu_median(lambda: O.avx2_matmul(14, x, raw, 1, 128256, 4096), 5)
        out["q6_k_gemv_128256x4096"] = {"value": round(algorithmic_bytes(14, 128256, 4096) / med / 1e9, 3),
                                        "unit": "GB/s", "cores": 1, "kind": "port", "cpu": host, "nproc": os.cpu_count(),
                                        "sample": "median of 5 full GEMVs (avx2::matmul_q6_k restated): %.1f ms"
                                                  % (med * 1e3)}
        print("[bench] cpu C3: %s" % out["q6_k_gemv_128256x4096"], file=sys.stderr, flush=True)
    for nn, (raw, a) in sorted(gemm.items()):
        t0 = time.perf_counter()
        O.avx2_matmul(12, a, raw, 512, nn, 4096)
        el = time.perf_counter() - t0
        out["q4_k_gemm_m512_n%d" % nn] = {"value": round(2.0 * 512 * nn * 4096 / el / 1e9, 3), "unit": "GFLOP/s",
                                          "cores": 1, "kind": "port", "cpu": host, "nproc": os.cpu_count(),
                                          "sample": "one m=512 call of avx2::matmul_q4_k restated: %.2f s" % el}
        print("[bench] cpu C4 n=%d: %s" % (nn, out["q4_k_gemm_m512_n%d" % nn]), file=sys.stderr, flush=True)
    if dec is not None:
        import numpy as np

        c = dec["cfg"]
        ocfg = O.LlamaCfg(c.vocab_size, c.d_model, c.num_layers, c.num_heads, c.num_kv_heads, c.head_dim, c.d_ff,
                          c.max_seq_len, c.rope_base, c.rms_norm_eps)
        s_, co = O.precompute_rope(c.max_seq_len, c.head_dim, c.rope_base)
        fill = dec["prefilled"]
        ts = []
        agree = 0
        for i, tok in enumerate(dec["tokens"]):
            t0 = time.perf_counter()
            logits, fill = O.decode_step(ocfg, dec["emb"][i], fill, dec["layers"], [12] * 7, dec["norms"],
                                         dec["final"], dec["lm"], 14, s_, co, dec["kv"], fill)
            ts.append(time.perf_counter() - t0)
            if i + 1 < len(dec["tokens"]):
                agree += int(O.argmax(logits) == dec["tokens"][i + 1])
        mean = sum(ts) / len(ts)
        out["decode_8b_q4k"] = {"value": round(1.0 / mean, 4), "unit": "tok/s", "cores": 1, "kind": "port",
                                "cpu": host, "nproc": os.cpu_count(),
                                "sample": "%d CPU decode steps of the 32-layer model after 2048 positions, mean %.2f s "
                                          "per token; greedy tokens equal to the GPU's on %d of %d steps"
                                          % (len(ts), mean, agree, len(ts) - 1)}
        print("[bench] cpu C5: %s" % out["decode_8b_q4k"], file=sys.stderr, flush=True)
    return out


def cpu_baseline(raw, x, n, k, seconds=10.0):
    """The oracle's AVX2-path restatement (single thread, as the reference's
    avx2::matmul_q4_k) timed on this host over repeated full GEMVs."""
    from oracle import oracle as O

    os.sched_setaffinity(0, {sorted(os.sched_getaffinity(0))[0]})
    calls = 0
    t0 = time.perf_counter()
    while True:
        O.avx2_matmul(12, x, raw, 1, n, k)
        calls += 1
        el = time.perf_counter() - t0
        if el >= seconds:
            break
    nbytes = algorithmic_bytes(12, n, k)
    return {"value": round(nbytes * calls / el / 1e9, 3), "unit": "GB/s", "cores": 1, "kind": "port",
            "cpu": cpu_name(), "nproc": os.cpu_count(),
            "sample": "%d full Q4_K GEMVs 14336x4096 (avx2::matmul_q4_k restated, oracle/oracle.c) in %.1f s on one "
                      "pinned core of a %d-thread host" % (calls, el, os.cpu_count() or 0)}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--no-extra", action="store_true", help="headline only")
    ap.add_argument("--extra",
                    default="floor,q8,q6,boundary,q5,dotprod,mfma,gemm,gemm_q8,gemm_q6k,gemm_q5k,gemm_q80,decode,q4_k_m,q8_0_model",
                    help="comma-separated extra sections to run: floor, q8, q6, boundary (host-slice calls; after q6), "
                         "q5, dotprod, gemm, gemm_q8, gemm_q6k, gemm_q5k, gemm_q80, "
                         "decode, q4_k_m, q8_0_model (default), f16, q2k (GGUF-order formats), decode_eager (the decode step "
                         "without its HIP graph; these three not run by default)")
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--calib-copy-mib", type=int, default=0,
                    help="also run one device-to-device copy of this many MiB (HBM counter calibration under rocprofv3)")
    args = ap.parse_args()
    if args.gpus != 1:
        print("bench.py: this build measures one GPU only; --gpus %d is not supported (run with --gpus 1)"
              % args.gpus, file=sys.stderr)
        sys.exit(2)

    import torch

    if not torch.cuda.is_available():
        print("bench.py: no GPU visible", file=sys.stderr)
        sys.exit(1)
    import aether_amd as A

    A.check(A.lib().aeth_init(0), "aeth_init")
    props = torch.cuda.get_device_properties(0)
    torch.cuda.synchronize()

    if args.calib_copy_mib:
        nb_ = args.calib_copy_mib << 20
        src = torch.empty(nb_, dtype=torch.uint8, device="cuda").fill_(1)
        dst = torch.empty_like(src)
        torch.cuda.synchronize()
        dst.copy_(src)
        torch.cuda.synchronize()
        print("[bench] calibration copy: %d bytes read, %d bytes written" % (nb_, nb_), file=sys.stderr, flush=True)
        del src, dst

    n, k = 14336, 4096
    head = bench_gemv(torch, A, 12, n, k, args.steps, args.warmup)
    print("[bench] Q4_K GEMV %dx%d: %.3f us  %.1f GB/s" % (n, k, head["ms"] * 1e3, head["gbs"]), file=sys.stderr,
          flush=True)
    extra = {}
    sections = set() if args.no_extra else set(x.strip() for x in args.extra.split(",") if x.strip())
    want_cpu = not args.no_cpu
    cpu_in = {"q8": None, "q6": None, "gemm": {}, "dec": None}
    q6_raw, q6_us = None, None
    if "floor" in sections:  # the plain read of the headline's weight bytes over 16 rotated buffers
        wbytes = n * (k // 256) * 144
        f = bench_read_floor(torch, A, wbytes, args.steps, args.warmup)
        extra["read_floor_33MB"] = {"GB/s": round(f["gbs"], 1), "us": round(f["ms"] * 1e3, 3),
                                    "frac_hbm": round(f["gbs"] / HBM_PEAK_GBS, 4), "bytes": wbytes,
                                    "headline_over_floor": round(head["ms"] / f["ms"], 4)}
        print("[bench] read floor: %s" % extra["read_floor_33MB"], file=sys.stderr, flush=True)
        lbytes = 128256 * 16 * 210  # the LM head's weight bytes (C3), two rotated buffers as its GEMV
        f = bench_read_floor(torch, A, lbytes, max(20, args.steps // 4), max(3, args.warmup // 4), copies=2)
        extra["read_floor_431MB"] = {"GB/s": round(f["gbs"], 1), "us": round(f["ms"] * 1e3, 3),
                                     "frac_hbm": round(f["gbs"] / HBM_PEAK_GBS, 4), "bytes": lbytes}
        print("[bench] read floor 431 MB: %s" % extra["read_floor_431MB"], file=sys.stderr, flush=True)
    if "q8" in sections:
        r = bench_gemv(torch, A, 8, 4096, 4096, args.steps, args.warmup, seed=0xAE7E41)
        extra["q8_0_gemv_4096x4096"] = {"GB/s": round(r["gbs"], 1), "us": round(r["ms"] * 1e3, 3),
                                         "frac_hbm": round(r["gbs"] / HBM_PEAK_GBS, 4),
                                         "traffic": profile_traffic("q8_0_gemv_4096x4096"),
                                         "parity": "scalar q8_0.rs (the reference's x86 AVX2 Q8_0 kernel reads "
                                                   "quants 16-23 for elements 8-15 and past the last block, "
                                                   "avx2.rs:163; its outputs differ from these)"}
        print("[bench] Q8_0 GEMV: %s" % extra["q8_0_gemv_4096x4096"], file=sys.stderr, flush=True)
        if want_cpu:
            cpu_in["q8"] = (r["raw0"].cpu().numpy(), r["x"].cpu().numpy())
        del r
    if "q6" in sections:
        r = bench_gemv(torch, A, 14, 128256, 4096, max(20, args.steps // 4), max(3, args.warmup // 4), copies=2,
                       seed=0xAE7E42)
        extra["q6_k_gemv_128256x4096"] = {"GB/s": round(r["gbs"], 1), "us": round(r["ms"] * 1e3, 3),
                                           "frac_hbm": round(r["gbs"] / HBM_PEAK_GBS, 4),
                                           "traffic": profile_traffic("q6_k_gemv_128256x4096")}
        print("[bench] Q6_K GEMV: %s" % extra["q6_k_gemv_128256x4096"], file=sys.stderr, flush=True)
        if want_cpu:
            cpu_in["q6"] = (r["raw0"].cpu().numpy(), r["x"].cpu().numpy())
        q6_raw, q6_us = r["raw0"], r["ms"] * 1e3
        del r
    if "boundary" in sections:  # host-slice calls through the plugin boundary, C2 and C3
        b2 = bench_boundary(torch, A, 12, n, k, head["raw0"], head["ms"] * 1e3)
        extra["boundary_q4_k_14336x4096"] = b2
        print("[bench] boundary C2: %s" % b2, file=sys.stderr, flush=True)
        if q6_raw is not None:
            b3 = bench_boundary(torch, A, 14, 128256, 4096, q6_raw, q6_us, calls=10)
            extra["boundary_q6_k_128256x4096"] = b3
            print("[bench] boundary C3: %s" % b3, file=sys.stderr, flush=True)
        A.lib().aeth_weight_cache_clear()
    if "q5" in sections:
        r = bench_gemv(torch, A, 13, 14336, 4096, args.steps, args.warmup, seed=0xAE7E44)
        extra["q5_k_gemv_14336x4096"] = {"GB/s": round(r["gbs"], 1), "us": round(r["ms"] * 1e3, 3),
                                          "frac_hbm": round(r["gbs"] / HBM_PEAK_GBS, 4)}
        print("[bench] Q5_K GEMV: %s" % extra["q5_k_gemv_14336x4096"], file=sys.stderr, flush=True)
    if "dotprod" in sections:  # the headline shape on the int8 dot-product path (a14 activations)
        r = bench_gemv(torch, A, 12, n, k, args.steps, args.warmup, seed=0xAE7E45, flags=A.MM_Q8_ACTIVATIONS)
        extra["q4_k_gemv_14336x4096_dotprod"] = {"GB/s": round(r["gbs"], 1), "us": round(r["ms"] * 1e3, 3),
                                                  "frac_hbm": round(r["gbs"] / HBM_PEAK_GBS, 4)}
        print("[bench] Q4_K GEMV dotprod: %s" % extra["q4_k_gemv_14336x4096_dotprod"], file=sys.stderr, flush=True)
    for sec, dt, nn, kk in (("f16", 1, 4096, 4096), ("q2k", 10, 4096, 4096)):
        if sec in sections:  # GGUF-order weights (quantized_matmul_impl's dequantize route)
            r = bench_gemv(torch, A, dt, nn, kk, args.steps, args.warmup, copies=8, seed=0xAE7E46)
            key = "%s_gguf_order_gemv_%dx%d" % ({1: "f16", 10: "q2_k"}[dt], nn, kk)
            extra[key] = {"GB/s": round(r["gbs"], 1), "us": round(r["ms"] * 1e3, 3),
                          "frac_hbm": round(r["gbs"] / HBM_PEAK_GBS, 4)}
            print("[bench] %s: %s" % (key, extra[key]), file=sys.stderr, flush=True)
    mfma = None
    if "mfma" in sections:  # the matrix-core rates this box sustains (the GEMM's measured roofline)
        mfma = {"fp16_TFLOP/s": round(bench_mfma_rate(torch, A, 0), 1),
                "int8_TOP/s": round(bench_mfma_rate(torch, A, 1), 1)}
        mfma["frac_of_spec"] = {"fp16": round(mfma["fp16_TFLOP/s"] / FP16_PEAK_TFLOPS, 4),
                                "int8": round(mfma["int8_TOP/s"] / INT8_PEAK_TOPS, 4)}
        extra["mfma_rate_measured"] = mfma
        print("[bench] MFMA rate: %s" % mfma, file=sys.stderr, flush=True)
    if "gemm" in sections:
        gsteps, gwarm = max(3, min(args.steps, 50)), max(1, min(args.warmup, 5))
        for nn in (4096, 14336):
            g = bench_gemm(torch, A, nn, 4096, 512, gsteps, gwarm)
            extra["q4_k_gemm_m512_n%d" % nn] = {"TFLOP/s": round(g["tflops"], 2), "ms": round(g["ms"], 4),
                                                 "frac_int8_peak": round(g["tflops"] / INT8_PEAK_TOPS, 4),
                                                 "frac_fp16_peak": round(g["tflops"] / FP16_PEAK_TFLOPS, 4),
                                                 "steps": gsteps, "mode": "exact (f32 activations)"}
            if mfma:  # the exact mode runs two fp16 MFMA passes per product: its ceiling is half the fp16 rate
                extra["q4_k_gemm_m512_n%d" % nn]["frac_exact_mode_ceiling"] = round(
                    g["tflops"] / (mfma["fp16_TFLOP/s"] / 2), 4)
            print("[bench] Q4_K GEMM n=%d: %s" % (nn, extra["q4_k_gemm_m512_n%d" % nn]), file=sys.stderr, flush=True)
            if want_cpu:
                cpu_in["gemm"][nn] = (g["raw0"].cpu().numpy(), g["a"].cpu().numpy())
            del g
    if "gemm_q8" in sections:  # the dot-product mode's GEMM: a14 Q8_0 activation blocks
        gsteps, gwarm = max(3, min(args.steps, 50)), max(1, min(args.warmup, 5))
        for nn in (4096, 14336):
            g = bench_gemm(torch, A, nn, 4096, 512, gsteps, gwarm, flags=A.MM_Q8_ACTIVATIONS)
            extra["q4_k_gemm_m512_n%d_q8act" % nn] = {"TFLOP/s": round(g["tflops"], 2), "ms": round(g["ms"], 4),
                                                       "frac_int8_peak": round(g["tflops"] / INT8_PEAK_TOPS, 4),
                                                       "steps": gsteps, "mode": "q8 (Q8_0 activation blocks)"}
            print("[bench] Q4_K GEMM q8 n=%d: %s" % (nn, extra["q4_k_gemm_m512_n%d_q8act" % nn]), file=sys.stderr,
                  flush=True)
            del g
    if "gemm_q6k" in sections:  # the Q6_K GEMM at a Q4_K_M file's attn_v / ffn_down shapes (and 4096 × 4096)
        for nn, kk in ((4096, 4096), (4096, 14336), (1024, 4096)):
            r = bench_batched(torch, A, 14, nn, kk, 512, max(3, min(args.steps, 20)), 2)
            key = "q6_k_gemm_m512_n%d_k%d" % (nn, kk)
            extra[key] = {"TFLOP/s": round(r["tflops"], 2), "ms": round(r["ms"], 4),
                          "path": "Q6_K GEMM: exact mode, three fp16 MFMA passes per product"}
            if mfma:  # three passes: the ceiling is a third of the fp16 rate
                extra[key]["frac_exact_mode_ceiling"] = round(r["tflops"] / (mfma["fp16_TFLOP/s"] / 3), 4)
            print("[bench] Q6_K GEMM m=512 n=%d k=%d: %s" % (nn, kk, extra[key]), file=sys.stderr, flush=True)
    if "gemm_q5k" in sections:  # the Q5_K GEMM (a Q5_K_M file's q, k, o, gate and up projections)
        for nn, kk in ((4096, 4096), (14336, 4096)):
            r = bench_batched(torch, A, 13, nn, kk, 512, max(3, min(args.steps, 20)), 2)
            key = "q5_k_gemm_m512_n%d_k%d" % (nn, kk)
            extra[key] = {"TFLOP/s": round(r["tflops"], 2), "ms": round(r["ms"], 4),
                          "path": "Q5_K GEMM: exact mode, two fp16 MFMA passes per product"}
            if mfma:
                extra[key]["frac_exact_mode_ceiling"] = round(r["tflops"] / (mfma["fp16_TFLOP/s"] / 2), 4)
            print("[bench] Q5_K GEMM m=512 n=%d k=%d: %s" % (nn, kk, extra[key]), file=sys.stderr, flush=True)
    if "gemm_q80" in sections:  # the Q8_0 GEMM (a Q8_0 file's prefill projections)
        for nn, kk in ((4096, 4096), (4096, 14336)):
            r = bench_batched(torch, A, 8, nn, kk, 512, max(3, min(args.steps, 20)), 2)
            key = "q8_0_gemm_m512_n%d_k%d" % (nn, kk)
            extra[key] = {"TFLOP/s": round(r["tflops"], 2), "ms": round(r["ms"], 4),
                          "path": "Q8_0 GEMM: exact mode, two fp16 MFMA passes per product"}
            if mfma:
                extra[key]["frac_exact_mode_ceiling"] = round(r["tflops"] / (mfma["fp16_TFLOP/s"] / 2), 4)
            print("[bench] Q8_0 GEMM m=512 n=%d k=%d: %s" % (nn, kk, extra[key]), file=sys.stderr, flush=True)
    if "q4_k_m" in sections:
        extra["q4_k_m_decode_prefill_8b"] = bench_q4_k_m(torch, A)
        print("[bench] Q4_K_M 8B: %s" % extra["q4_k_m_decode_prefill_8b"], file=sys.stderr, flush=True)
    if "q8_0_model" in sections:  # every layer weight Q8_0 (prefill on the Q8_0 GEMM, decode on the Q8_0 GEMV)
        extra["q8_0_decode_prefill_8b"] = bench_q4_k_m(torch, A, layer_dtypes=(8,) * 7,
                                                       mix="Q8_0 layer weights; LM head Q6_K")
        print("[bench] Q8_0 8B: %s" % extra["q8_0_decode_prefill_8b"], file=sys.stderr, flush=True)
    if "decode" in sections:
        d = bench_decode(torch, A, want_cpu=want_cpu)
        cpu_in["dec"] = d.pop("cpu_model")
        extra["decode_8b_q4k"] = {"tok/s": round(d["tok_s"], 1), "ms_per_token": round(d["ms_per_token"], 4),
                                  "GB/s": round(d["gbs"], 1), "frac_hbm": round(d["gbs"] / HBM_PEAK_GBS, 4),
                                  "tokens": 128, "prefilled": 2048, "first_tokens": d["first_tokens"]}
        print("[bench] decode 8B: %s" % extra["decode_8b_q4k"], file=sys.stderr, flush=True)
        extra["prefill_8b_q4k_512"] = {"tok/s": round(d["prefill_tok_s"], 1), "ms": round(d["prefill_ms"], 2),
                                       "TFLOP/s": round(d["prefill_tflops"], 2), "tokens": 512}
        print("[bench] prefill 8B: %s" % extra["prefill_8b_q4k_512"], file=sys.stderr, flush=True)
        extra["prefill_8b_q4k_32"] = {"tok/s": round(32 / d["prefill32_ms"] * 1e3, 1), "ms": round(d["prefill32_ms"], 3),
                                      "tokens": 32}
        print("[bench] prefill 8B, 32 tokens: %s" % extra["prefill_8b_q4k_32"], file=sys.stderr, flush=True)

    if "decode_eager" in sections:  # not a default section: the same decode without the HIP graph
        d = bench_decode_eager(torch, A, n_tokens=max(2, min(args.steps, 128)))
        extra["decode_8b_q4k_eager"] = {"tok/s": round(d["tok_s"], 1), "ms_per_token": round(d["ms_per_token"], 4),
                                        "tokens": d["tokens"], "prefilled": 2048, "first_tokens": d["first_tokens"]}
        print("[bench] decode 8B eager: %s" % extra["decode_8b_q4k_eager"], file=sys.stderr, flush=True)

    cpu = None
    if not args.no_cpu:
        raw = head["raw0"].cpu().numpy()
        x = head["x"].cpu().numpy()
        cpu_par = cpu_rows_parallel(raw, x, n, k)  # before the single-core leg pins this process
        print("[bench] cpu, scalar kernel over threads: %s" % cpu_par, file=sys.stderr, flush=True)
        extra["cpu_q4_k_gemv_rows_parallel"] = cpu_par
        cpu = cpu_baseline(raw, x, n, k, args.cpu_seconds)  # pins this process to one core
        print("[bench] cpu baseline: %s" % cpu, file=sys.stderr, flush=True)
        for key, val in cpu_configs(cpu_in["q8"], cpu_in["q6"], cpu_in["gemm"], cpu_in["dec"]).items():
            extra.setdefault(key, {})["cpu_baseline"] = val

    out = {
        "metric": "Q4_K GEMV HBM GB/s (% peak); prefill GEMM TFLOP/s; 8B-shape decode tok/s",
        "value": round(head["gbs"], 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(head["ms"], 6),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "q4_k x f32 (int8-digit dot, f32 accumulate)",
        "data": "synthetic (seeded device generator per BASELINE configs; 16 rotated weight copies)",
        "config": {"workload": "Q4_K GEMV batch 1, weight 14336x4096, x f32[4096] (BASELINE configs[1])",
                   "n": n, "k": k, "weight_copies": 16, "device": props.name, "cus": props.multi_processor_count},
        "roofline": {"bound": "hbm", "achieved": round(head["gbs"], 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(head["gbs"] / HBM_PEAK_GBS, 4), "traffic": measured_traffic()},
        "cpu_baseline": cpu,
        "extra": extra,
    }
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
