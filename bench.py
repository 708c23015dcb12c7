"""Benchmark: exact Q8_0 greedy decode at Mistral-7B shape on one MI355X.

The workload is the Mistral-7B-shape decode: 32 mistral-dense layers
(hidden 4096, 32 query / 8 KV heads of 128, SwiGLU 14336, vocab 32000,
RoPE base 1e6), random-init Q8_0 weights from a seed, a 512-token prompt and
greedy decoding at batch 1. One step is one decode pass (every layer and the
head over one row, then the greedy selection); the timed region is `--steps`
consecutive steps after the prompt pass, timed with HIP events on the
session's stream (the weights and KV cache are already resident in HBM).

The JSON line also carries:
- roofline: the metric's Q8_0 GEMV (M=1, K=4096, N=14336) timed with HIP
  events over launches that cycle through enough copies of the matrix that
  each one reads from HBM; algorithmic bytes = weights at 34/32 B each +
  activations + outputs;
- decode_roofline: the whole decode step against HBM (weights + KV cache
  read per token);
- teacher_forced: the 2048-row teacher-forced chain pass on the same model
  (device time of the pass; wall time with the per-layer SHA-256
  checkpoints) and its gate|up product (M=2048, K=4096, N=28672) on the
  int8 matrix cores, against the 5.0 POP/s dense int8 peak (the executed
  MFMA work counts each signed byte digit plane of the activations);
- pcie_inclusive: the drop-in entry point q8gpu_product (host buffers in
  and out of every call, as the reference's gpu.rs calls it) timed per call
  for the microbenchmark's GEMV and GEMM, the matrix already uploaded;
- cpu_baseline: the CPU oracle (a C restatement of the reference's kernels)
  timed on a bounded sample of the same decode on this host's cores;
- measured_peaks: the part's HBM read rate (a plain streaming kernel over
  1 GiB) and int8 matrix-core rate (independent 32x32x32 MFMAs, constant
  and random operands), beside the vendor figures the fractions use.
"""
from __future__ import annotations

import argparse
import ctypes as C
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "decode tokens/sec + Q8 GEMV HBM GB/s (% peak), bit-exact, 1 MI355X"
PEAK_HBM_GBPS = 8000.0
# HBM bytes one launch of the roofline GEMV moves, from rocprofv3 FETCH_SIZE
# and WRITE_SIZE passes scaled by a 256 MiB device copy (fetch x2.000, write
# x1.000): profiles/q8_gemv_row_scale_k4096_n14336.md. Re-measure when the
# kernel or its layout changes.
GEMV_TRAFFIC_BYTES = 59_372_000
PROMPT = 512  # the prompt length of the timed workload
DECODE_TOKENS = 512
TEACHER_FORCED_ROWS = 2048


def log(msg):
    print(msg, file=sys.stderr, flush=True)


def gemv_roofline(decode_timing):
    """The metric's GEMV: M=1, K=4096, N=14336, weights one f16 scale per row."""
    g = decode_timing.time_gemv()
    achieved = g["algorithmic_bytes"] / (g["us"] * 1e-6) / 1e9
    return {"bound": "hbm", "achieved": round(achieved, 1), "peak": PEAK_HBM_GBPS, "unit": "GB/s",
            "frac": round(achieved / PEAK_HBM_GBPS, 4), "traffic": GEMV_TRAFFIC_BYTES,
            "kernel": "q8_gemv_persistent<row scale>", "launch": "Q8_0 GEMV M=1 K=4096 N=14336",
            "algorithmic_bytes": g["algorithmic_bytes"], "avg_launch_us": round(g["us"], 3)}


def cpu_baseline(model, threads, steps=4):
    """The oracle (a C restatement of the reference's CPU kernels, OpenMP
    over rows as the reference's rayon is) on this host, after every GPU
    measurement, on bounded samples of each workload:
    - decode: `steps` steps at positions 512.. over a random-filled KV cache
      (the 512-token prompt pass is not run), on `threads` threads, and one
      step on one thread;
    - the two products of the microbenchmark: the M=1 GEMV (K=4096,
      N=14336, row scales) and the M=512 GEMM (K=N=4096), on `threads`;
    - the teacher-forced pass: one layer over the first 256 of the 2048 rows
      (positions 0..255), reported in rows per second."""
    from oracle import cpu
    run = cpu.OracleRun(model, PROMPT + steps + 2, threads=threads)
    rng = np.random.default_rng(5)
    for layer in range(model.num_layers):
        run.k_cache[layer][:PROMPT] = rng.integers(-(1 << 18), 1 << 18, run.k_cache[layer][:PROMPT].shape)
        run.v_cache[layer][:PROMPT] = rng.integers(-(1 << 18), 1 << 18, run.v_cache[layer][:PROMPT].shape)
    tok = 1
    t0 = time.perf_counter()
    for i in range(steps):
        rows, _ = run.pass_rows([tok], PROMPT + i)
        logits = run.logits(rows[-1])
        tok = int(np.argmax(logits))
    dt = time.perf_counter() - t0
    # one step on one thread
    run.threads = 1
    t0 = time.perf_counter()
    rows, _ = run.pass_rows([tok], PROMPT + steps)
    run.logits(rows[-1])
    dt1 = time.perf_counter() - t0
    run.threads = threads

    from iris_amd import synth
    k, n = 4096, 14336
    w = synth.q8_matrix(synth.tensor_seed(2, 1), n, k, synth.scale_base_for(k), True)
    x1 = rng.integers(-127, 128, (1, k)).astype(np.int32) * 300
    cpu.linear_q8(x1, w, threads)
    t0 = time.perf_counter()
    for _ in range(5):
        cpu.linear_q8(x1, w, threads)
    gemv_us = (time.perf_counter() - t0) / 5 * 1e6
    w2 = synth.q8_matrix(synth.tensor_seed(4, 1), 4096, 4096, synth.scale_base_for(4096), True)
    x2 = rng.integers(-(1 << 20), 1 << 20, (512, 4096)).astype(np.int32)
    t0 = time.perf_counter()
    cpu.linear_q8(x2, w2, threads)
    gemm_us = (time.perf_counter() - t0) * 1e6

    tf_rows = 256
    tf = cpu.OracleRun(model, tf_rows, threads=threads)
    from iris_amd import decode_timing
    ids = synth.token_ids(decode_timing.PROMPT_SEED, tf_rows, model.vocab)
    x = tf.embed(list(ids))
    t0 = time.perf_counter()
    tf.layer_pass(0, x, 0)
    tf_s = time.perf_counter() - t0
    return {"value": round(steps / dt, 4), "unit": "tokens/s", "cores": threads, "kind": "port",
            "sample": f"{steps} decode steps of the same model at positions {PROMPT}..{PROMPT + steps - 1} "
                      f"over a random-filled KV cache (CPU oracle, {threads} threads; prompt pass not run)",
            "single_thread": {"value": round(1.0 / dt1, 4), "unit": "tokens/s", "cores": 1,
                              "sample": f"one decode step at position {PROMPT + steps}"},
            "gemv_us": {"value": round(gemv_us, 1), "cores": threads,
                        "sample": "Q8_0 GEMV M=1 K=4096 N=14336 (row scales), mean of 5"},
            "gemm_us": {"value": round(gemm_us, 1), "cores": threads,
                        "sample": "Q8_0 GEMM M=512 K=4096 N=4096 (row scales), one product"},
            "teacher_forced_layer": {"value": round(tf_rows / tf_s, 1), "unit": "rows/s", "cores": threads,
                                     "ms_per_layer_2048_rows_linear": round(tf_s * 1e3 * 2048 / tf_rows, 1),
                                     "sample": f"layer 0 over rows 0..{tf_rows - 1} of the 2048-row pass "
                                               "(attention grows with the rows, so 2048 rows take longer "
                                               "than the linear figure)"}}


def main():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=DECODE_TOKENS - 1)
    ap.add_argument("--warmup", type=int, default=8)
    ap.add_argument("--cpu-steps", type=int, default=4)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--direct-launches", action="store_true",
                    help="time the decodes launch by launch instead of as graph replays (for kernel traces)")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one MI355X: the library has no multi-GPU path (run with --gpus 1)",
              file=sys.stderr)
        sys.exit(2)
    if args.steps < 1 or PROMPT + args.steps > 4096:
        print("--steps must be in 1..3584", file=sys.stderr)
        sys.exit(2)

    from iris_amd import decode_timing, native, synth

    if not args.direct_launches and native.kernel_tracer_loaded():
        # The library refuses graph replays under a kernel tracer.
        log("kernel tracer loaded: timing the decodes launch by launch")
        args.direct_launches = True
    decode_timing.USE_GRAPH = not args.direct_launches
    native.check(native.lib().q8gpu_init(), "q8gpu_init")
    bench = decode_timing.DecodeBench(max(args.steps, args.warmup), log=log)
    if args.warmup:
        bench.run(args.warmup)
    native.check(native.lib().q8gpu_synchronize(), "synchronize")
    wall0 = time.perf_counter()
    ms_per_token, prefill_ms, tokens = bench.run(args.steps)
    native.check(native.lib().q8gpu_synchronize(), "synchronize")
    wall = time.perf_counter() - wall0
    log(f"decode {ms_per_token:.3f} ms/token; prompt pass {prefill_ms:.1f} ms; wall {wall:.2f}s")

    # Determinism: the same decode again gives the same tokens.
    _, _, tokens2 = bench.run(min(args.steps, 32))
    deterministic = tokens2 == tokens[:len(tokens2)]

    per_token = bench.bytes_per_step(args.steps)
    decode_gbps = per_token / (ms_per_token * 1e-3) / 1e9

    roof = gemv_roofline(decode_timing)
    log(f"GEMV {roof['avg_launch_us']} us = {roof['achieved']} GB/s ({100 * roof['frac']:.1f}% of peak)")
    peaks = decode_timing.measured_peaks()
    roof["frac_of_measured_stream"] = round(roof["achieved"] / peaks["hbm_read_gbps"], 4)
    log(f"measured peaks: HBM read {peaks['hbm_read_gbps']} GB/s; int8 MFMA {peaks['mfma_i8_tops_constant']} TOP/s "
        f"constant operands, {peaks['mfma_i8_tops_random']} random")
    gpb = decode_timing.time_gemv(per_row_scale=False)
    gemv_pb = {"launch": "Q8_0 GEMV M=1 K=4096 N=14336, one f16 scale per block",
               "avg_launch_us": round(gpb["us"], 3), "algorithmic_bytes": gpb["algorithmic_bytes"],
               "achieved": round(gpb["algorithmic_bytes"] / (gpb["us"] * 1e-6) / 1e9, 1), "unit": "GB/s"}
    gemv_pb["frac"] = round(gemv_pb["achieved"] / PEAK_HBM_GBPS, 4)
    log(f"GEMV per-block scales {gemv_pb['avg_launch_us']} us = {gemv_pb['achieved']} GB/s")

    # The teacher-forced chain pass (2048 rows, per-layer checkpoint hashes)
    # on the same model, and its largest product on the int8 matrix cores.
    bench.session.free()
    tf = decode_timing.time_teacher_forced_session(bench.dm, bench.vocab, TEACHER_FORCED_ROWS)
    log(f"teacher-forced {TEACHER_FORCED_ROWS} rows: pass {tf['pass_ms']} ms, with checkpoints {tf['checkpoint_ms']} ms")
    bench.dm.free()
    gemm = decode_timing.time_gemm(TEACHER_FORCED_ROWS)
    gemm["frac_of_measured_random"] = round(gemm["mfma_tops"] / peaks["mfma_i8_tops_random"], 4)
    log(f"MFMA GEMM {gemm['shape']}: {gemm['us']} us = {gemm['mfma_tops']} TOP/s ({100 * gemm['frac']:.1f}% of int8 peak)")
    # The isolated product microbenchmark's GEMM: M=512, K=N=4096, row scales,
    # activations a * s_t (a in [-127, 127], s_t = 2^8 + random % 2^8).
    c2 = decode_timing.time_gemm(512, n=4096, k=4096, x=decode_timing.c2_activations())
    c2["algorithmic_frac"] = round(c2["product_tops"] / decode_timing.INT8_PEAK_TOPS, 4)
    log(f"C2 GEMM {c2['shape']}: {c2['us']} us, {c2['digit_planes']} digit planes = {c2['mfma_tops']} TOP/s issued "
        f"({100 * c2['frac']:.1f}%), {c2['product_tops']} TOP/s algorithmic ({100 * c2['algorithmic_frac']:.1f}%)")
    # The drop-in entry point's PCIe-inclusive rate (host buffers in and out
    # of every call), for both microbenchmark products.
    host_gemv = decode_timing.time_host_product(1)
    host_gemm = decode_timing.time_host_product(512, n=4096, k=4096, x=decode_timing.c2_activations())
    pcie = {"entry_point": "q8gpu_product (host activations in, host outputs out, synchronous)",
            "gemv_us": host_gemv["us"], "gemm_us": host_gemm["us"], "gemv_shape": "M=1 K=4096 N=14336",
            "gemm_shape": "M=512 K=4096 N=4096", "gemm_host_bytes": host_gemm["host_bytes"]}
    log(f"q8gpu_product with host buffers: GEMV {host_gemv['us']} us per call, GEMM M=512 {host_gemm['us']} us")
    gemm_pb = decode_timing.time_gemm(TEACHER_FORCED_ROWS, per_row_scale=False)
    log(f"MFMA GEMM per-block scales {gemm_pb['shape']}: {gemm_pb['us']} us, {gemm_pb['weight_planes']} weight planes "
        f"= {gemm_pb['mfma_tops']} TOP/s ({100 * gemm_pb['frac']:.1f}% of int8 peak)")

    # The Gemma-2B-shape decode (a 128-token prompt, then 255 timed steps).
    gb = decode_timing.GemmaDecodeBench(255, log=log)
    gb.run(8)
    g_ms, g_pre, _ = gb.run(255)
    g_bytes = gb.bytes_per_step(255)
    gb.free()
    g_gbps = g_bytes / (g_ms * 1e-3) / 1e9
    gemma = {"workload": "gemma-2b-shape Q8_0 greedy decode, prompt 128 + 256 tokens, batch 1",
             "tokens_per_s": round(1e3 / g_ms, 2), "ms_per_step": round(g_ms, 4), "prompt_pass_ms": round(g_pre, 2),
             "bytes_per_token": int(g_bytes), "achieved": round(g_gbps, 1), "unit": "GB/s",
             "frac": round(g_gbps / PEAK_HBM_GBPS, 4)}
    log(f"gemma-2b decode {g_ms:.3f} ms/token ({gemma['tokens_per_s']} tokens/s, {g_gbps:.0f} GB/s)")

    base = None
    if not args.no_cpu:
        threads = int(os.environ.get("OMP_NUM_THREADS", os.cpu_count() or 1))
        base = cpu_baseline(synth.mistral_7b(seed=decode_timing.MISTRAL_7B_SEED), threads, args.cpu_steps)
        log(f"CPU oracle: {base['value']} tokens/s on {threads} threads, {base['single_thread']['value']} on 1; "
            f"GEMV {base['gemv_us']['value']} us, GEMM M=512 {base['gemm_us']['value']} us; "
            f"teacher-forced layer {base['teacher_forced_layer']['value']} rows/s")

    line = {
        "metric": METRIC, "value": round(1000.0 / ms_per_token, 2), "unit": "tokens/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(ms_per_token, 4),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "i8xi32->i64 exact",
        "data": "synthetic (random-init Q8_0 weights from a seed, uniform prompt ids)",
        "config": {"workload": "mistral-7b-shape Q8_0 greedy decode, prompt 512 + 512 tokens, batch 1",
                   "prompt_tokens": PROMPT, "decode_steps_timed": args.steps, "batch": 1,
                   "decode_launches": "direct" if args.direct_launches else "graph replay"},
        "roofline": roof,
        "measured_peaks": peaks,
        "gemv_per_block": gemv_pb,
        "c2_gemm": c2,
        "pcie_inclusive": pcie,
        "decode_roofline": {"bound": "hbm", "achieved": round(decode_gbps, 1), "peak": PEAK_HBM_GBPS,
                            "unit": "GB/s", "frac": round(decode_gbps / PEAK_HBM_GBPS, 4),
                            "bytes_per_token": int(per_token)},
        "prompt_pass_ms": round(prefill_ms, 2),
        "gemma_2b_decode": gemma,
        "deterministic_rerun": deterministic,
        "teacher_forced": dict(tf, workload="mistral-7b-shape chain pass over 2048 uniform ids, "
                                            "per-layer SHA-256 checkpoints", mfma_gemm=gemm,
                                 mfma_gemm_per_block=gemm_pb),
        "cpu_baseline": base,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
