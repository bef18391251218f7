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
int8 dot-product path (and, on request, GGUF-order F16 / Q2_K GEMVs), plus
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
    stream = torch.cuda.current_stream()
    for i in range(warmup):
        fn(i)
    torch.cuda.synchronize()
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
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


def bench_gemm(torch, A, n, k, m, steps, warmup, seed=0xAE7E43):
    L = A.lib()
    copies = 2
    ws, _ = make_weights(torch, A, 12, n, k, copies, seed)
    a = torch.empty(m * k, dtype=torch.float32, device="cuda")
    A.check(L.aeth_fill_normal_f32(seed ^ 0x77, a.data_ptr(), m * k, 0.0, 1.0, None))
    c = torch.empty(m * n, dtype=torch.float32, device="cuda")
    s = torch.cuda.current_stream().cuda_stream

    def step(i):
        A.check(L.aeth_qmatmul(ws[i % copies], a.data_ptr(), m, c.data_ptr(), 0, s), "gemm")

    ms = time_launches(torch, step, steps, warmup)
    for w in ws:
        L.aeth_weight_free(w)
    return {"ms": ms, "tflops": 2.0 * m * n * k / (ms * 1e-3) / 1e12}


def bench_decode(torch, A, n_tokens=128, prefilled=2048, prefill_tokens=512):
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
            "prefill_tok_s": prefill_tokens / pf_s, "prefill_ms": pf_s * 1e3, "prefill_tflops": pf_flops / pf_s / 1e12}


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
            "kind": "port (scalar kernel, rows over threads)",
            "sample": "%d full Q4_K GEMVs 14336x4096 in %.1f s" % (calls, el)}


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
            "sample": "%d full Q4_K GEMVs 14336x4096 (avx2::matmul_q4_k restated, oracle/oracle.c) in %.1f s on %s"
                      % (calls, el, platform.processor() or platform.machine())}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--no-extra", action="store_true", help="headline only")
    ap.add_argument("--extra", default="q8,q6,q5,dotprod,gemm,decode",
                    help="comma-separated extra sections to run: q8, q6, q5, dotprod, gemm, decode (default), "
                         "f16, q2k (GGUF-order formats, not run by default)")
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
    if "q8" in sections:
        r = bench_gemv(torch, A, 8, 4096, 4096, args.steps, args.warmup, seed=0xAE7E41)
        extra["q8_0_gemv_4096x4096"] = {"GB/s": round(r["gbs"], 1), "us": round(r["ms"] * 1e3, 3),
                                         "frac_hbm": round(r["gbs"] / HBM_PEAK_GBS, 4)}
        print("[bench] Q8_0 GEMV: %s" % extra["q8_0_gemv_4096x4096"], file=sys.stderr, flush=True)
    if "q6" in sections:
        r = bench_gemv(torch, A, 14, 128256, 4096, max(20, args.steps // 4), max(3, args.warmup // 4), copies=2,
                       seed=0xAE7E42)
        extra["q6_k_gemv_128256x4096"] = {"GB/s": round(r["gbs"], 1), "us": round(r["ms"] * 1e3, 3),
                                           "frac_hbm": round(r["gbs"] / HBM_PEAK_GBS, 4)}
        print("[bench] Q6_K GEMV: %s" % extra["q6_k_gemv_128256x4096"], file=sys.stderr, flush=True)
        del r
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
    if "gemm" in sections:
        for nn in (4096, 14336):
            g = bench_gemm(torch, A, nn, 4096, 512, 5, 2)
            extra["q4_k_gemm_m512_n%d" % nn] = {"TFLOP/s": round(g["tflops"], 2), "ms": round(g["ms"], 4),
                                                 "frac_int8_peak": round(g["tflops"] / INT8_PEAK_TOPS, 4)}
            print("[bench] Q4_K GEMM n=%d: %s" % (nn, extra["q4_k_gemm_m512_n%d" % nn]), file=sys.stderr, flush=True)
    if "decode" in sections:
        d = bench_decode(torch, A)
        extra["decode_8b_q4k"] = {"tok/s": round(d["tok_s"], 1), "ms_per_token": round(d["ms_per_token"], 4),
                                  "GB/s": round(d["gbs"], 1), "frac_hbm": round(d["gbs"] / HBM_PEAK_GBS, 4),
                                  "tokens": 128, "prefilled": 2048, "first_tokens": d["first_tokens"]}
        print("[bench] decode 8B: %s" % extra["decode_8b_q4k"], file=sys.stderr, flush=True)
        extra["prefill_8b_q4k_512"] = {"tok/s": round(d["prefill_tok_s"], 1), "ms": round(d["prefill_ms"], 2),
                                       "TFLOP/s": round(d["prefill_tflops"], 2), "tokens": 512}
        print("[bench] prefill 8B: %s" % extra["prefill_8b_q4k_512"], file=sys.stderr, flush=True)

    cpu = None
    if not args.no_cpu:
        raw = head["raw0"].cpu().numpy()
        x = head["x"].cpu().numpy()
        cpu_par = cpu_rows_parallel(raw, x, n, k)  # before the single-core leg pins this process
        print("[bench] cpu, scalar kernel over threads: %s" % cpu_par, file=sys.stderr, flush=True)
        extra["cpu_q4_k_gemv_rows_parallel"] = cpu_par
        cpu = cpu_baseline(raw, x, n, k, args.cpu_seconds)
        print("[bench] cpu baseline: %s" % cpu, file=sys.stderr, flush=True)

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
