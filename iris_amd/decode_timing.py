"""Device-side timing of the exact decode loop and of its Q8_0 GEMV.

Both measurements run entirely on the GPU with HIP events on the stream the
kernels are launched on; the weights, KV cache and activations are resident
in HBM before the timed region starts.

`python -m iris_amd.decode_timing [--steps K] [--warmup W]` prints one JSON
line with the same figures the benchmark reports, so the kernels it launches
can be traced on their own (for example under `rocprofv3 --kernel-trace
--stats`).
"""
from __future__ import annotations

import argparse
import ctypes as C
import json
import sys

import numpy as np

from . import native, synth
from .direct import DeviceModel, Session

PROMPT = 512
# The timed decodes replay the step as a HIP graph (True) or issue its
# launches one by one (False: the same kernels and time, and what a kernel
# tracer follows without intercepting graph launches).
USE_GRAPH = True
MISTRAL_7B_SEED = 0x7B7B
PROMPT_SEED = 0x5EED
# Q8_0 bytes of every product one decode step reads at Mistral-7B shape:
# 32 x (q|k|v 6144 + o 4096 + gate|up 28672 + down 4096 rows) x K + head.
MISTRAL_7B_WEIGHT_BYTES = 7554793472

GEMV_N, GEMV_K = 14336, 4096


def gemv_algorithmic_bytes(n: int = GEMV_N, k: int = GEMV_K) -> int:
    """Q8_0 weights (34 bytes per 32 values) + i32 activations + i32 outputs."""
    return n * k * 34 // 32 + k * 4 + n * 4


def copy_calibration(mib: int = 256, repeats: int = 3) -> int:
    """Device-to-device copies of `mib` MiB, `repeats` times: a plain copy
    kernel of known size (each dispatch reads and writes exactly mib MiB),
    against which hardware byte counters such as FETCH_SIZE and WRITE_SIZE
    are scaled."""
    n = mib << 20
    src, dst = native.DeviceBuffer(n), native.DeviceBuffer(n)
    for _ in range(repeats):
        native.check(native.lib().iris_memcpy_d2d(dst.ptr, src.ptr, n), "copy")
    return n


def time_gemv(iterations: int = 200, n: int = GEMV_N, k: int = GEMV_K, per_row_scale: bool = True) -> dict:
    """Average duration of one Q8_0 GEMV launch (M=1) with one f16 scale per
    row (or per block: the device reads one f16 per block beside the
    weights). Launches cycle through enough copies of the matrix (more than
    600 MB in all) that each reads its weights from HBM, not from the 256 MB
    Infinity Cache."""
    from .tensor import Q8Matrix

    raw = synth.q8_matrix(synth.tensor_seed(2, 1), n, k, synth.scale_base_for(k), per_row_scale)
    copies = max(1, -(-600_000_000 // (n * k * 34 // 32)))
    mats = [Q8Matrix.from_bytes(raw, n, k) for _ in range(copies)]
    arr = (C.c_void_p * copies)(*[m.handle.value for m in mats])
    rng = np.random.default_rng(2)
    x = (rng.integers(-127, 128, (1, k)) * (256 + int(rng.integers(0, 256)))).astype(np.int32)
    dx = native.DeviceBuffer.from_array(x)
    dout = native.DeviceBuffer(n * 4)
    ms = C.c_double()
    native.check(native.lib().iris_time_product(arr, copies, dx.ptr, 1, dout.ptr, iterations, C.byref(ms)),
                 "time GEMV")
    for m in mats:
        m.free()
    return {"us": ms.value * 1e3, "copies": copies, "n": n, "k": k,
            "algorithmic_bytes": gemv_algorithmic_bytes(n, k)}


def time_host_product(tokens: int, n: int = GEMV_N, k: int = GEMV_K, iterations: int = 20,
                      x: np.ndarray | None = None) -> dict:
    """Wall time per call of the drop-in entry point q8gpu_product (host
    activations in, host outputs out, synchronous: the calls the reference's
    gpu.rs makes), the matrix (one f16 scale per row) already on the device,
    after one untimed call that sizes the library's device arena: the
    PCIe-inclusive rate of a product."""
    import time
    from .tensor import Q8Matrix, linear_slab_from_source

    raw = synth.q8_matrix(synth.tensor_seed(2, 1), n, k, synth.scale_base_for(k), True)
    m = Q8Matrix.from_bytes(raw, n, k)
    m.prepare_matrix_cores()  # a per-block scale matrix is folded for the matrix cores
    if x is None:
        rng = np.random.default_rng(2)
        x = (rng.integers(-127, 128, (tokens, k)) * (256 + int(rng.integers(0, 256)))).astype(np.int32)
    linear_slab_from_source(x, m)
    t0 = time.perf_counter()
    for _ in range(iterations):
        linear_slab_from_source(x, m)
    us = (time.perf_counter() - t0) / iterations * 1e6
    m.free()
    return {"us": round(us, 1), "tokens": tokens, "n": n, "k": k,
            "host_bytes": int(tokens * k * 4 + tokens * n * 4), "calls": iterations}


INT8_PEAK_TOPS = 5000.0  # MI355X dense int8 MFMA


def digit_planes_needed(x: np.ndarray, group: int = 128) -> np.ndarray:
    """Signed byte digits each group of `group` tokens takes on the matrix
    cores: the most any value of the group needs (the bytes of v +
    0x8080808080, each xor 0x80; 1 to 5)."""
    d = (x.astype(np.int64) + 0x8080808080).astype(np.uint64) ^ np.uint64(0x8080808080)
    limbs = np.ones(d.shape, dtype=np.int64)
    for sh in (8, 16, 24, 32):
        limbs = np.maximum(limbs, np.where((d >> np.uint64(sh)) != 0, sh // 8 + 1, 1))
    per_token = limbs.max(axis=1)
    return np.array([per_token[i:i + group].max() for i in range(0, len(per_token), group)])


def c2_activations(tokens: int = 512, k: int = GEMV_K, seed: int = 5) -> np.ndarray:
    """The isolated product's activations: a * s_t with a uniform in
    [-127, 127] and a per-token Q16.16 integer s_t = 2^8 + (random % 2^8)."""
    rng = np.random.default_rng(seed)
    a = rng.integers(-127, 128, (tokens, k)).astype(np.int64)
    s_t = (256 + rng.integers(0, 256, (tokens, 1))).astype(np.int64)
    return (a * s_t).astype(np.int32)


def time_gemm(tokens: int = 2048, n: int = 14336 * 2, k: int = GEMV_K, iterations: int = 20,
              magnitude_bits: int = 21, per_row_scale: bool = True, x=None) -> dict:
    """Average duration of one multi-token Q8_0 product on the int8 matrix
    cores (digit planes + MFMA GEMM) at the gate|up shape of the 2048-row
    pass, with activations of `magnitude_bits` bits (three signed byte
    digits for the default, as the normalised inputs of that pass have).
    The matrix-core work is 2 * tokens * n * k per digit plane of the
    activations, times the weight digit planes of a per-block scale matrix
    (its scales folded into the weights: one f16 per block, the reference
    bundles' base + random significand layout)."""
    from .tensor import Q8Matrix

    raw = synth.q8_matrix(synth.tensor_seed(3, 1), n, k, synth.scale_base_for(k), per_row_scale)
    m = Q8Matrix.from_bytes(raw, n, k)
    m.prepare_matrix_cores()  # a per-block scale matrix is folded for the matrix cores
    if x is None:
        rng = np.random.default_rng(4)
        half = 1 << (magnitude_bits - 1)
        x = rng.integers(-half, half, (tokens, k)).astype(np.int32)
    dx = native.DeviceBuffer.from_array(np.ascontiguousarray(x, dtype=np.int32))
    dout = native.DeviceBuffer(tokens * n * 4)
    L = native.lib()
    ws_bytes = L.q8gpu_workspace_bytes(m.handle, tokens)
    ws = native.DeviceBuffer(ws_bytes)
    ms = C.c_double()
    native.check(L.iris_time_product_ws(m.handle, dx.ptr, tokens, dout.ptr, ws.ptr, ws_bytes, iterations,
                                        C.byref(ms)), "time GEMM")
    info = m.info()
    m.free()
    # digit planes of each 128-token group (as the launch takes them)
    groups = digit_planes_needed(x)
    sizes = np.minimum(128, tokens - 128 * np.arange(len(groups)))
    digits = int(groups.max())
    # weight digit planes: 1 for a row-scale matrix; a folded one holds
    # (device bytes - int8 weights - f16 scales - row shifts) / int8 weights
    qs = n * k
    wplanes = 1 if per_row_scale else round((info["bytes"] - qs - n * k // 32 * 2 - 4 * ((n + 15) // 16 * 16)) / qs)
    ops = 2.0 * float((groups * sizes).sum()) * n * k * wplanes
    tops = ops / (ms.value * 1e-3) / 1e12
    return {"shape": f"M={tokens} K={k} N={n}", "scales": "per row" if per_row_scale else "per block (folded)",
            "us": round(ms.value * 1e3, 1), "digit_planes": digits, "weight_planes": wplanes,
            "mfma_tops": round(tops, 1), "peak_tops": INT8_PEAK_TOPS, "frac": round(tops / INT8_PEAK_TOPS, 4),
            "product_tops": round(2.0 * tokens * n * k / (ms.value * 1e-3) / 1e12, 1)}


def time_teacher_forced_session(dm, vocab: int, rows: int = 2048, repeats: int = 2) -> dict:
    """The teacher-forced pass of every layer over `rows` uniform-random ids
    on an uploaded model: device time of the pass (HIP events), and the wall
    time of the per-layer checkpoint call (pass, rows to pinned host memory,
    one SHA-256 per layer), after one untimed call that sets up its staging."""
    import time
    session = Session(dm, rows, rows)
    ids = synth.token_ids(PROMPT_SEED, rows, vocab)
    device_ms = min(session.time_pass(ids) for _ in range(repeats))
    _, hashes = session.layer_pass(ids, keep_rows=False)
    t = time.perf_counter()
    _, hashes2 = session.layer_pass(ids, keep_rows=False)
    wall_ms = (time.perf_counter() - t) * 1e3
    session.free()
    return {"rows": rows, "pass_ms": round(device_ms, 2), "checkpoint_ms": round(wall_ms, 2),
            "rows_per_s": round(rows / (wall_ms * 1e-3), 1), "layers": len(hashes),
            "repeatable": hashes2 == hashes, "last_layer_sha256": hashes[-1]}


class DecodeBench:
    """Mistral-7B-shape model on the device with a session sized for a
    512-token prompt followed by `max_steps` decode steps."""

    def __init__(self, max_steps: int, log=None):
        import time
        log = log or (lambda msg: None)
        t = time.time()
        model = synth.mistral_7b(seed=MISTRAL_7B_SEED)
        log(f"weights generated in {time.time() - t:.1f}s")
        t = time.time()
        self.dm = DeviceModel(model)
        log(f"uploaded in {time.time() - t:.1f}s")
        self.shape = model.shape
        self.vocab = model.vocab
        del model.tensors  # the device holds the weights now
        self.session = Session(self.dm, PROMPT + max_steps + 1, PROMPT)
        self.prompt = synth.token_ids(PROMPT_SEED, PROMPT, self.vocab)

    def run(self, steps: int):
        """(ms per decode step, prompt-pass ms, token ids) for one timed
        decode of `steps` steps after the prompt pass."""
        return self.session.time_decode(self.prompt, steps, use_graph=USE_GRAPH)

    def bytes_per_step(self, steps: int) -> float:
        """HBM bytes one decode step must read: every weight once plus the
        K and V caches up to the step's position (averaged over the run)."""
        s = self.shape
        kvw = s.num_key_value_heads * s.head_dim
        mean_ctx = PROMPT + (steps + 1) / 2.0
        return MISTRAL_7B_WEIGHT_BYTES + 2 * 4 * kvw * s.num_hidden_layers * mean_ctx


GEMMA_2B_SEED = 0x2B2B
GEMMA_PROMPT = 128


def decode_step_bytes(model) -> int:
    """Bytes of weights one decode step reads, from the model's tensors: every
    layer matrix and the head as Q8_0 (34 bytes per 32 weights), the Q16.16
    matrices (PLE gate and projection, the per-layer model projection) at 4
    bytes a value, and one embedding row per table (the selected token's)."""
    from .model import PREFIX
    total = 0
    for name, t in model.tensors.items():
        if not name.startswith(PREFIX + "layers.") and name not in (PREFIX + "lm_head.weight",
                                                                    PREFIX + "per_layer_model_projection.weight"):
            continue
        total += t.nbytes
    if model.shape.tied_head:
        total += model.tensors[PREFIX + "embed_tokens.weight"].nbytes
    for table in (PREFIX + "embed_tokens.weight", PREFIX + "embed_tokens_per_layer.weight"):
        if table in model.tensors:
            total += model.tensors[table].shape[1]
    return int(total)


class GemmaDecodeBench:
    """The Gemma-2B-shape model (18 layers, hidden 2048, 8 heads of 256 on
    one KV head, GeGLU 16384, vocab 256000, PLE 256, softcap 30, tied head)
    on the device, a 128-token prompt and `max_steps` decode steps."""

    def __init__(self, max_steps: int, log=None):
        import time
        log = log or (lambda msg: None)
        t = time.time()
        model = synth.gemma_2b(seed=GEMMA_2B_SEED)
        log(f"gemma-2b weights generated in {time.time() - t:.1f}s")
        self.weight_bytes = decode_step_bytes(model)
        self.dm = DeviceModel(model)
        self.shape = model.shape
        self.layers = model.num_layers
        self.head_dims = [model.head_dim_at(layer) for layer in range(model.num_layers)]
        del model.tensors
        self.session = Session(self.dm, GEMMA_PROMPT + max_steps + 1, GEMMA_PROMPT)
        self.prompt = synth.token_ids(PROMPT_SEED, GEMMA_PROMPT, self.shape.vocab_size)

    def run(self, steps: int):
        return self.session.time_decode(self.prompt, steps, use_graph=USE_GRAPH)

    def bytes_per_step(self, steps: int) -> float:
        """Weights (decode_step_bytes) plus every layer's K and V up to the
        step's position, averaged over the run."""
        mean_ctx = GEMMA_PROMPT + (steps + 1) / 2.0
        kv = sum(2 * 4 * self.shape.num_key_value_heads * hd for hd in self.head_dims)
        return self.weight_bytes + kv * mean_ctx

    def free(self):
        self.session.free()
        self.dm.free()


def time_teacher_forced(rows: int = 2048, repeats: int = 2, log=None, per_row_scale: bool = True) -> dict:
    """time_teacher_forced_session on a freshly uploaded Mistral-7B-shape model."""
    log = log or (lambda msg: None)
    model = synth.mistral_7b(seed=MISTRAL_7B_SEED, per_row_scale=per_row_scale)
    dm = DeviceModel(model)
    vocab = model.vocab
    del model.tensors
    log("model on device")
    r = time_teacher_forced_session(dm, vocab, rows, repeats)
    dm.free()
    return r


def trace_decode(steps: int = 64) -> dict:
    """A short decode for kernel traces: a session of 1024 positions, a
    512-token prompt (ids from seed 1), `steps` greedy steps (graph replays,
    or launch by launch under a kernel tracer), timed with HIP events;
    nothing else runs."""
    model = synth.mistral_7b(seed=MISTRAL_7B_SEED)
    dm = DeviceModel(model)
    del model.tensors
    session = Session(dm, 1024, PROMPT)
    ms, prefill, _ = session.time_decode(synth.token_ids(1, PROMPT, 32000), steps, use_graph=USE_GRAPH)
    session.free()
    dm.free()
    return {"decode_ms_per_step": round(ms, 4), "prompt_pass_ms": round(prefill, 2), "steps": steps}


def eager_decode(steps: int, gemma: bool = False) -> dict:
    """A short decode with every launch issued from the host (no graph), for
    kernel traces and counters: Mistral-7B shape after a 512-token prompt
    (session of 1024 positions), or Gemma-2B shape after a 128-token prompt;
    returns the wall time of the generate call."""
    import time
    if gemma:
        g = GemmaDecodeBench(steps)
        session, prompt = g.session, g.prompt
    else:
        model = synth.mistral_7b(seed=MISTRAL_7B_SEED)
        dm = DeviceModel(model)
        del model.tensors
        session, prompt = Session(dm, 1024, PROMPT), synth.token_ids(1, PROMPT, 32000)
    t = time.time()
    out = session.generate(prompt, steps, use_graph=False)
    wall = time.time() - t
    if gemma:
        g.free()
    else:
        session.free()
        dm.free()
    return {"family": "gemma-dense" if gemma else "mistral-dense", "steps": steps, "tokens": len(out.token_ids),
            "wall_s": round(wall, 3)}


def measured_peaks(stream_bytes: int = 1 << 30) -> dict:
    """The part's measured peaks, beside the vendor figures (8 TB/s HBM,
    5.0 POP/s dense int8): the read rate of a plain streaming kernel over
    `stream_bytes` (four times the last-level cache, so every pass comes
    from HBM), and the int8 matrix-core rate of a loop of independent
    32x32x32 MFMAs with constant operands and with random operands that
    change every instruction (the matrix cores' clock drops under switching
    operands; the exact products' operands are random)."""
    L = native.lib()
    buf = native.DeviceBuffer(stream_bytes)
    native.check(L.iris_memcpy_h2d(buf.ptr, np.zeros(1 << 20, dtype=np.uint8).ctypes.data, 1 << 20), "fill")
    gbps = C.c_double()
    native.check(L.iris_probe_hbm_read(buf.ptr, stream_bytes, 20, C.byref(gbps)), "HBM read probe")
    buf.free()
    out = {"hbm_read_gbps": round(gbps.value, 1), "hbm_stream_bytes": stream_bytes}
    for name, rnd in (("mfma_i8_tops_constant", 0), ("mfma_i8_tops_random", 1)):
        t = C.c_double()
        native.check(L.iris_probe_mfma_i8(rnd, 20000, C.byref(t)), "MFMA probe")
        out[name] = round(t.value, 1)
    return out


def handoff_latencies(sizes=(8, 32, 288, 1024)) -> dict:
    """What a kernel pays to wait on other workgroups, against a launch
    boundary: a flag's round trip between workgroups on two XCDs, one
    dependent agent-scope atomic add, and arrival barriers of `sizes`
    workgroups on one counter (last arrival to last release)."""
    L = native.lib()
    out = {}
    for g in sizes:
        rt, at, bar = C.c_double(), C.c_double(), C.c_double()
        native.check(L.iris_probe_handoff(g, C.byref(rt), C.byref(at), C.byref(bar)), "handoff probe")
        out["flag_round_trip_us"] = round(rt.value, 3)
        out["atomic_add_us"] = round(at.value, 3)
        out[f"barrier_{g}_workgroups_us"] = round(bar.value, 2)
    return out


def row_latencies(floods=(0, 1, 3, 7)) -> dict:
    """How long a product's activation-row load takes behind the weight
    stream: median microseconds of a vector load (the staged products' row
    path) and of a scalar load (the broadcast products' digit planes) while
    `floods` other waves of each CU's workgroup keep 16 cold loads per lane
    in flight."""
    L = native.lib()
    out = {}
    for f in floods:
        v, sc = C.c_double(), C.c_double()
        native.check(L.iris_probe_row_latency(f, C.byref(v), C.byref(sc)), "row latency probe")
        out[f"vector_load_behind_{f}_waves_us"] = round(v.value, 2)
        out[f"scalar_load_behind_{f}_waves_us"] = round(sc.value, 2)
    return out


def main(argv=None):
    ap = argparse.ArgumentParser(description="time the exact decode loop and its GEMV on the GPU")
    ap.add_argument("--steps", type=int, default=PROMPT - 1)
    ap.add_argument("--warmup", type=int, default=8)
    ap.add_argument("--gemv-only", action="store_true", help="time only the Q8_0 GEMV")
    ap.add_argument("--calibrate", action="store_true",
                    help="first run a 256 MiB device-to-device copy (byte-counter calibration)")
    ap.add_argument("--pass-rows", type=int, default=0,
                    help="time only the teacher-forced pass over this many rows")
    ap.add_argument("--gemm-only", action="store_true", help="time only the MFMA product at the gate|up shape")
    ap.add_argument("--c2-gemm", action="store_true",
                    help="time only the isolated product's GEMM (M=512, K=N=4096, row scales)")
    ap.add_argument("--per-block", action="store_true",
                    help="with --gemm-only, --gemv-only or --pass-rows: per-block scale matrices")
    ap.add_argument("--trace-decode", type=int, default=0, metavar="STEPS",
                    help="only a short decode of STEPS steps (for kernel traces)")
    ap.add_argument("--gemma-2b", type=int, default=0, metavar="STEPS",
                    help="only the Gemma-2B-shape decode: a 128-token prompt and STEPS timed steps")
    ap.add_argument("--eager-decode", type=int, default=0, metavar="STEPS",
                    help="only a decode of STEPS steps launched from the host, no graph (for traces and "
                         "counters); Mistral-7B shape, or Gemma-2B shape with --gemma")
    ap.add_argument("--gemma", action="store_true", help="with --eager-decode: the Gemma-2B shape")
    ap.add_argument("--peaks", action="store_true",
                    help="only the measured peaks: HBM read stream and int8 MFMA (constant and random operands), "
                         "the handoff latencies between workgroups, and a row load's latency behind the "
                         "weight stream")
    args = ap.parse_args(argv)
    global USE_GRAPH
    if USE_GRAPH and native.kernel_tracer_loaded():
        # The library refuses graph replays under a kernel tracer.
        print("kernel tracer loaded: decodes launched one by one", file=sys.stderr, flush=True)
        USE_GRAPH = False
    native.check(native.lib().q8gpu_init(), "q8gpu_init")
    if args.peaks:
        print(json.dumps(measured_peaks()), flush=True)
        print(json.dumps(handoff_latencies()), flush=True)
        print(json.dumps(row_latencies()), flush=True)
        return
    if args.eager_decode:
        print(json.dumps(eager_decode(args.eager_decode, args.gemma)), flush=True)
        return
    if args.trace_decode:
        print(json.dumps(trace_decode(args.trace_decode)), flush=True)
        return
    if args.gemma_2b:
        g = GemmaDecodeBench(args.gemma_2b, log=lambda m: print(m, file=sys.stderr, flush=True))
        g.run(8)
        ms, prefill, _ = g.run(args.gemma_2b)
        b = g.bytes_per_step(args.gemma_2b)
        print(json.dumps({"decode_ms_per_step": round(ms, 4), "tokens_per_s": round(1e3 / ms, 1),
                          "prompt_pass_ms": round(prefill, 2), "bytes_per_step": int(b),
                          "achieved_gbps": round(b / (ms * 1e-3) / 1e9, 1)}), flush=True)
        g.free()
        return
    if args.c2_gemm:
        print(json.dumps(time_gemm(512, n=4096, k=GEMV_K, x=c2_activations())), flush=True)
        return
    if args.gemm_only:
        print(json.dumps(time_gemm(per_row_scale=not args.per_block)), flush=True)
        return
    if args.pass_rows:
        r = time_teacher_forced(args.pass_rows, log=lambda m: print(m, file=sys.stderr, flush=True),
                                per_row_scale=not args.per_block)
        print(json.dumps(r), flush=True)
        return
    if args.calibrate:
        copy_calibration()
    if args.gemv_only:
        g = time_gemv(per_row_scale=not args.per_block)
        print(json.dumps({"gemv_us": round(g["us"], 3), "gemv_copies": g["copies"],
                          "algorithmic_bytes": g["algorithmic_bytes"]}), flush=True)
        return
    bench = DecodeBench(max(args.steps, args.warmup), log=lambda m: print(m, file=sys.stderr, flush=True))
    if args.warmup:
        bench.run(args.warmup)
    ms, prefill, _ = bench.run(args.steps)
    g = time_gemv()
    print(json.dumps({"decode_ms_per_step": round(ms, 4), "prompt_pass_ms": round(prefill, 2),
                      "gemv_us": round(g["us"], 3), "gemv_copies": g["copies"]}), flush=True)


if __name__ == "__main__":
    main()
