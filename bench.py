#!/usr/bin/env python3
"""Benchmark of the quantized-matmul hot path on one MI355X.

Workload ("INT4 decode GEMV sweep over TinyLlama-1.1B
linear shapes"): one step is the 155 INT4 GEMVs (M=1) of one TinyLlama-1.1B
decode token -- 22 layers x {q 2048x2048, k 2048x256, v 2048x256,
o 2048x2048, gate 2048x5632, up 2048x5632, down 5632x2048} + lm_head
2048x32000 -- each layer with its own weight buffers (646.5 MB of codes and
scales per step, more than the 256 MB Infinity Cache, so weights stream from
HBM).  Weights are N(0, 0.02) fp32 packed on the GPU by vm_hip_pack_int4
(bit-exact with quant.cpp); each layer holds a device copy of its shape's
packed matrix at its own address.  Activations are N(0, 1) fp32.

Timed region: K graph replays of the captured step on one stream, bracketed
by HIP events and device synchronisation.  ``value`` is algorithmic bytes
(codes + scales + fp32 A + fp32 C, each once) per second over the region.
``roofline`` covers the dominant kernel (the shape whose launches take the
most time per step): its algorithmic bytes per launch over its average
launch duration, from a HIP graph of that shape's launches replayed between
two events on the launch stream.  ``cpu_baseline``
times the oracle's scalar INT4 path (src/cpu/ops/quantized_matmul.cpp:48-141)
on one pinned core over a bounded sample of the same step.

``grouped_sweep`` is the same 155 GEMVs with the siblings that read one
activation vector (q | k | v, gate | up) grouped into one launch each, as
the graph compiler groups them on DeviceType::HIP: 89 launches per step.
``value`` stays the per-QuantizedMatMul sweep.

``per_shape``, ``gemm`` and ``config1_int8_gemv`` time each launch on the
next of enough weight copies to walk >= 512 MB (twice the Infinity Cache),
so that their GB/s are HBM figures.

``config1_int8_gemv`` is BASELINE config 1, the INT8 per-column decode GEMV
at K 576 x N 1536, with its CPU leg: the oracle's restatement of the
reference's AVX2 streaming decode (quantized_matmul.cpp:146-188) on one
pinned core.

``gemm`` is BASELINE config 3, the MFMA path (M in {16, 128, 512}, K 2048,
N 5632, INT8 and INT4): TFLOP/s as a fraction of the dense fp16 MFMA peak
(2.5 PFLOP/s) and algorithmic GB/s.

``gemv_large`` runs the same GEMV kernel at 70B-class shapes (150-660 MB
per launch) where latency no longer dominates: GB/s and fraction of HBM
peak, showing what the kernel sustains once a launch is long enough.

``e2e`` adds the metric's second half, TinyLlama INT4 decode tokens/s
(512-token prompt, 256 greedy tokens) and SmolLM2-360M
INT8 (config 4: 128 + 128), on the resident HIP decoder with synthetic
weights: prefill and decode tokens/s, and the decode step's weight stream
(packed codes + scales of every QuantizedMatMul per token) as GB/s and as a
fraction of HBM peak.  ``persistent_step`` is the same decode with the
one-launch step vm_hip_decode_step (slower than the default captured
launch-per-projection step on this GPU, so reported beside it).  For
config 4, ``graph_engine`` is the drop-in path: the reference engine's loop
over a Graph on DeviceType::HIP per call, over config 4's 128 decode tokens,
with the reference layer's default attention chain and with its
use_fused_attention form, and the host time per step split into graph
construction, Graph::build, execute and the logits' readback.

Prints one JSON line.  Only --gpus 1 is supported (one GPU per box).
"""
from __future__ import annotations

import argparse
import ctypes
import json
import os
import sys
import time

import numpy as np
from ctypes import c_void_p

ROOT = os.path.dirname(os.path.abspath(__file__))
for _p in (os.path.join(ROOT, "velo-mind_amd"), os.path.join(ROOT, "oracle")):
    if _p not in sys.path:
        sys.path.insert(0, _p)

HBM_PEAK_GBS = 8000.0
LAYERS = 22
LAYER_SHAPES = [("q", 2048, 2048), ("k", 2048, 256), ("v", 2048, 256), ("o", 2048, 2048),
                ("gate", 2048, 5632), ("up", 2048, 5632), ("down", 5632, 2048)]
LM_HEAD = ("lm_head", 2048, 32000)
BLOCK = 32
METRIC = "qmatmul HBM GB/s (% of ~8 TB/s peak); TinyLlama INT4 decode tokens/sec"


def algo_bytes(k: int, n: int, m: int = 1) -> int:
    """Codes + fp32 scales + fp32 A + fp32 C, each counted once."""
    nb = (k + BLOCK - 1) // BLOCK
    return ((k + 1) // 2) * n + nb * n * 4 + m * k * 4 + m * n * 4


def step_shapes():
    shapes = []
    for layer in range(LAYERS):
        for name, k, n in LAYER_SHAPES:
            shapes.append((f"L{layer}.{name}", k, n))
    shapes.append(LM_HEAD)
    return shapes


def log(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


class Workload:
    """Device-resident weights, activations and outputs for one decode step."""

    def __init__(self, H, stream):
        self.H = H
        self.stream = stream
        rng = np.random.default_rng(20240601)
        self.masters = {}
        distinct = {(k, n) for _, k, n in LAYER_SHAPES} | {(LM_HEAD[1], LM_HEAD[2])}
        for k, n in sorted(distinct):
            w = (rng.standard_normal((k, n), dtype=np.float32) * np.float32(0.02)).astype(np.float32)
            dw = H.DeviceBuffer.from_array(w)
            packed = H.DeviceBuffer(((k + 1) // 2) * n)
            scales = H.DeviceBuffer(((k + BLOCK - 1) // BLOCK) * n * 4)
            H.pack_int4(dw.addr, packed.addr, scales.addr, k, n, BLOCK)
            H.synchronize()
            dw.close()
            self.masters[(k, n)] = (packed, scales)
        self.x = {k: H.DeviceBuffer.from_array(rng.standard_normal(k, dtype=np.float32)) for k in (2048, 5632)}
        self.out = {n: H.DeviceBuffer(n * 4) for n in (256, 2048, 5632, 32000)}
        # every GEMV of the step reads its own copy of the weights
        self.calls = []
        lib = H.open_library()
        for name, k, n in step_shapes():
            mp, ms = self.masters[(k, n)]
            if name == LM_HEAD[0]:
                p, s = mp, ms
            else:
                p = H.DeviceBuffer(mp.nbytes)
                s = H.DeviceBuffer(ms.nbytes)
                H.check(lib.vm_hip_memcpy_d2d(p.ptr, mp.ptr, mp.nbytes, stream.handle))
                H.check(lib.vm_hip_memcpy_d2d(s.ptr, ms.ptr, ms.nbytes, stream.handle))
            self.calls.append((name, k, n, p, s))
        stream.synchronize()
        self.bytes_per_step = sum(algo_bytes(k, n) for _, k, n, _, _ in self.calls)
        self.group_out = {}

    def launch_step(self) -> None:
        H, st = self.H, self.stream
        for _, k, n, p, s in self.calls:
            H.qmm_f32(self.x[k].addr, p.addr, s.addr, self.out[n].addr, 1, k, n, H.QUANT_INT4, BLOCK, st)

    def grouped_calls(self):
        """The same step with the siblings that read one activation vector
        grouped as the HIP graph compiler groups them (q | k | v and
        gate | up per layer): [(k, [(codes, scales, out, n), ...]), ...]."""
        groups, i = [], 0
        while i < len(self.calls):
            name, k, n, p, s = self.calls[i]
            part = name.split(".")[-1]
            size = {"q": 3, "gate": 2}.get(part, 1)
            members = []
            for name2, k2, n2, p2, s2 in self.calls[i:i + size]:
                out = self.group_out.setdefault(name2.split(".")[-1], self.H.DeviceBuffer(n2 * 4))
                members.append((p2.addr, s2.addr, out.addr, n2))
            groups.append((k, members))
            i += size
        return groups

    def launch_grouped_step(self, groups) -> None:
        H, st = self.H, self.stream
        for k, members in groups:
            H.qmm_group_f32(self.x[k].addr, 1, k, members, H.QUANT_INT4, BLOCK, st)


ROTATION_BYTES = 512 << 20   # weight copies a timed replay walks: twice the 256 MB Infinity Cache


class Rotation:
    """`copies` device copies of one packed weight (codes, scales) in one
    allocation, enough that a replay walking them reads at least
    ROTATION_BYTES, so that every launch streams its weights from HBM rather
    than from the Infinity Cache of the previous replay."""

    def __init__(self, H, codes, scales, stream, min_copies: int = 1, copies: int = 0):
        lib = H.open_library()
        self.cb, self.sb = codes.nbytes, scales.nbytes
        self.stride = (self.cb + self.sb + 255) // 256 * 256
        self.copies = copies or max(min_copies, -(-ROTATION_BYTES // (self.cb + self.sb)))
        self.buf = H.DeviceBuffer(self.copies * self.stride)
        base = self.buf.addr
        for i in range(self.copies):
            H.check(lib.vm_hip_memcpy_d2d(c_void_p(base + i * self.stride), codes.ptr, self.cb, stream.handle))
            H.check(lib.vm_hip_memcpy_d2d(c_void_p(base + i * self.stride + self.cb), scales.ptr, self.sb,
                                          stream.handle))
        stream.synchronize()
        self.addrs = [(base + i * self.stride, base + i * self.stride + self.cb) for i in range(self.copies)]
        self.bytes = self.copies * (self.cb + self.sb)

    def close(self) -> None:
        self.buf.close()


def timed_replay(H, stream, launch_all, reps: int, use_graph: bool = True) -> float:
    """Milliseconds per replay of launch_all, as one HIP graph (or eager
    launches) replayed `reps` times between two events on `stream`."""
    g = None
    if use_graph:
        g = H.Graph(stream)
        g.begin()
        launch_all()
        g.end()
    replay = g.launch if g is not None else launch_all
    replay()
    stream.synchronize()
    e0, e1 = H.Event(), H.Event()
    e0.record(stream.handle)
    for _ in range(reps):
        replay()
    e1.record(stream.handle)
    e1.synchronize()
    if g is not None:
        g.close()
    return e0.elapsed_ms(e1) / reps


def per_shape_durations(H, wl: Workload, reps: int, use_graph: bool) -> dict:
    """Average launch duration per shape: each shape's GEMV launched once
    per weight copy of a Rotation (>= 512 MB of copies, so every launch
    reads HBM), the launches replayed `reps` times between two events on
    the launch stream as one HIP graph (or, with use_graph False, as eager
    launches, which the host's launch rate can bound)."""
    st = wl.stream
    out = {}
    for key in sorted({(k, n) for _, k, n, _, _ in wl.calls}):
        calls = [c for c in wl.calls if (c[1], c[2]) == key]
        count = len(calls)
        k, n = key
        mp, ms = wl.masters[key]
        rot = Rotation(H, mp, ms, st)

        def launch_all():
            for pa, sa in rot.addrs:
                H.qmm_f32(wl.x[k].addr, pa, sa, wl.out[n].addr, 1, k, n, H.QUANT_INT4, BLOCK, st)

        out[key] = (timed_replay(H, st, launch_all, reps, use_graph) / rot.copies, count, rot.copies, rot.bytes)
        rot.close()
    return out


def measured_traffic(shape: str):
    """HBM bytes per launch of the GEMV of `shape` ("KxN") from the committed
    rocprofv3 counter summary profiles/gemv_int4_<shape>_traffic.md, whose
    line "traffic_bytes_per_launch: N" is FETCH_SIZE + WRITE_SIZE per
    dispatch scaled by the counters' reading of a plain copy of known size;
    (None, None) when no summary exists for the shape."""
    path = os.path.join(ROOT, "profiles", f"gemv_int4_{shape}_traffic.md")
    try:
        with open(path) as f:
            for line in f:
                if line.startswith("traffic_bytes_per_launch:"):
                    return int(line.split(":", 1)[1]), os.path.relpath(path, ROOT)
    except (OSError, ValueError):
        pass
    return None, None


def cpu_baseline(target_s: float) -> dict:
    """Oracle scalar INT4 GEMV (reference CPU algorithm), one pinned core."""
    import oracle as O

    rng = np.random.default_rng(7)
    mats = {}
    for _, k, n in LAYER_SHAPES + [LM_HEAD]:
        if (k, n) not in mats:
            w = (rng.standard_normal((k, n), dtype=np.float32) * np.float32(0.02)).astype(np.float32)
            p, s = O.quantize_int4(w, BLOCK)
            mats[(k, n)] = (p.view(np.int8), s, rng.standard_normal((1, k), dtype=np.float32))
    shapes = step_shapes()
    cpu = sorted(os.sched_getaffinity(0))[0]
    prev = os.sched_getaffinity(0)
    os.sched_setaffinity(0, {cpu})
    try:
        done_bytes = 0
        sweeps = 0
        t0 = time.perf_counter()
        # whole decode-step sweeps until the bounded sample time is reached
        while True:
            for _, k, n in shapes:
                p, s, x = mats[(k, n)]
                O.qmm(x, p, s, k, O.QUANT_INT4, BLOCK)
                done_bytes += algo_bytes(k, n)
            sweeps += 1
            if time.perf_counter() - t0 >= target_s:
                break
        dt = time.perf_counter() - t0
    finally:
        os.sched_setaffinity(0, prev)
    model, flags = "", set()
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name") and not model:
                    model = line.split(":", 1)[1].strip()
                elif line.startswith("flags") and not flags:
                    flags = set(line.split(":", 1)[1].split())
    except OSError:
        pass
    return {"value": round(done_bytes / dt / 1e9, 4), "unit": "GB/s", "cores": 1, "kind": "port",
            "host": {"nproc": os.cpu_count(), "model": model, "avx2": "avx2" in flags, "fma": "fma" in flags},
            "sample": f"{sweeps} full decode-step sweep(s) (155 INT4 GEMVs, M=1) of the oracle's scalar "
                      f"INT4 loop (src/cpu/ops/quantized_matmul.cpp:48-141), {dt:.1f} s on core {cpu}",
            "tokens_per_s": round(sweeps / dt, 4)}


# The drop-in path (graph engine) is timed on config 4's full workload
# (128-token prompt, 128 decode tokens), with the reference layer's default
# attention chain and with its use_fused_attention form.
GRAPH_ENGINE_E2E = {"smollm2_360m_int8": 128}

E2E_MODELS = {
    # TinyLlama-1.1B shapes, synthetic INT4 weights,
    # 512-token uniform-random prompt, 256 greedy decode tokens.
    "tinyllama_1.1b_int4": dict(cfg=dict(vocab_size=32000, hidden_size=2048, intermediate_size=5632, num_layers=22,
                                         num_heads=32, num_kv_heads=4, rms_norm_eps=1e-5, rope_theta=10000.0),
                                quant=2, block=32, prompt=512, steps=256),
    # SmolLM2-360M shapes, synthetic INT8 weights,
    # 128-token prompt, 128 greedy decode tokens; tied embeddings (the
    # lm_head is quant.cpp's INT8 packing of the embedding's transpose).
    "smollm2_360m_int8": dict(cfg=dict(vocab_size=49152, hidden_size=960, intermediate_size=2560, num_layers=32,
                                       num_heads=15, num_kv_heads=5, rms_norm_eps=1e-5, rope_theta=100000.0,
                                       tie_word_embeddings=True),
                              quant=1, block=0, prompt=128, steps=128, tied=True),
}


def decode_weight_bytes(c: dict, quant: int, block: int) -> int:
    """Packed codes + scales the decode step streams per token: every
    linear of every layer plus lm_head (QuantizedMatMul weights only)."""
    h, i, d = c["hidden_size"], c["intermediate_size"], c["hidden_size"] // c["num_heads"]
    kv = c["num_kv_heads"] * d
    shapes = [(h, h), (h, kv), (h, kv), (h, h), (h, i), (h, i), (i, h)] * c["num_layers"] + [(h, c["vocab_size"])]
    tot = 0
    for k, n in shapes:
        if quant == 2:
            tot += ((k + 1) // 2) * n + ((k + block - 1) // block) * n * 4
        else:
            tot += k * n + n * 4
    return tot


DECODE_PATHS = {0: "graph", 1: "per-op", 2: "slices", 3: "persistent"}


def e2e_bench(name: str, use_graph: bool = True, persistent: bool = False, graph_engine: bool = False,
              steps: int = 0, fused_attention: bool = False) -> dict:
    """Greedy generation on the resident HIP decoder (HIP-graph decode
    steps, or with persistent=True the one-launch step vm_hip_decode_step;
    device-event timing of the prefill and of the decode steps), or with
    graph_engine=True on the drop-in path: the reference engine's loop
    (llama_engine.cpp:333-455), one Graph on DeviceType::HIP built and run
    per call, host argmax over the logits read back, host wall-clock
    timing."""
    from velomind_hip import llama as VL

    spec = E2E_MODELS[name]

    class Cfg:
        pass

    cfg = Cfg()
    for k, v in spec["cfg"].items():
        setattr(cfg, k, v)
    w = VL.Weights(cfg)
    w.fill_synthetic(20240601, 0.02)
    if spec.get("tied"):
        w.tie_lm_head()
    steps = steps or spec["steps"]
    if graph_engine:
        sess = VL.Session(w, VL.ENGINE_GRAPH, spec["quant"], spec["block"], fused_attention=fused_attention)
    else:
        prev = os.environ.get("VELOMIND_DECODE_PERSISTENT")
        os.environ["VELOMIND_DECODE_PERSISTENT"] = "1" if persistent else "0"
        try:
            sess = VL.Session(w, VL.ENGINE_RESIDENT, spec["quant"], spec["block"],
                              max_seq=spec["prompt"] + max(steps, 8) + 1)
        finally:
            if prev is None:
                del os.environ["VELOMIND_DECODE_PERSISTENT"]
            else:
                os.environ["VELOMIND_DECODE_PERSISTENT"] = prev
    path = DECODE_PATHS[sess.decode_path()]
    if persistent and path != "persistent":
        raise RuntimeError(f"{name}: the persistent decode step does not cover this shape (path {path})")
    prompt = np.random.default_rng(5).integers(0, cfg.vocab_size, spec["prompt"]).astype(np.int32)
    sess.generate(prompt, 8 if not graph_engine else 2, use_hip_graph=use_graph)  # warm-up (sizes workspaces)
    _, (pf_s, dec_s, nd) = sess.generate(prompt, steps, use_hip_graph=use_graph)
    step_ms = sess.step_timing() if graph_engine else None
    wb = decode_weight_bytes(spec["cfg"], spec["quant"], spec["block"])
    dec_tps = nd / dec_s
    out = {"prompt_tokens": spec["prompt"], "decode_tokens": steps, "decode_steps_timed": nd,
           "prefill_tokens_per_s": round(spec["prompt"] / pf_s, 1), "prefill_ms": round(pf_s * 1e3, 3),
           "decode_tokens_per_s": round(dec_tps, 1), "decode_us_per_token": round(dec_s / nd * 1e6, 1),
           "decode_weight_bytes_per_token": wb, "decode_weight_GB_s": round(wb * dec_tps / 1e9, 1),
           "decode_frac_of_hbm_peak": round(wb * dec_tps / 1e9 / HBM_PEAK_GBS, 4),
           "weights": ("int4 block 32" if spec["quant"] == 2 else "int8 per column") +
                      ", synthetic N(0, 0.02), packed on the GPU",
           "decode_path": path,
           "engine": ("graph engine: a Graph on DeviceType::HIP per call (the drop-in Op path), host argmax, "
                      "host wall-clock timing" if graph_engine else
                      "resident HIP decoder, " + ("HIP-graph" if use_graph else "eager") +
                      " decode steps, greedy argmax on device")}
    if step_ms is not None:
        out["host_ms_per_step"] = {k: round(v, 3) for k, v in step_ms.items() if k != "steps"}
        # Each step's graph is built on a helper thread while the previous
        # step executes: the main thread waiting for it means the host's
        # construction + build + teardown, not the device, set the rate.
        out["bound"] = "host (graph construction and build)" if step_ms["wait_ms"] > 0.05 else "device"
        out["attention"] = "FusedAttention (use_fused_attention)" if fused_attention else \
            "MatMul / Softmax / MatMul chain (the reference default)"
    sess.close()
    w.close()
    return out


def decode_trace_report(tokens: int = 8) -> dict:
    """Phase timing of the one-launch decode step (TinyLlama-1.1B INT4,
    512-token prompt) from a library built with VELOMIND_DECODE_TRACE=1:
    the timestamps of the last step's phases (decode_persistent.hip lists
    the events), as medians over workgroups and layers, and the chain of
    one middle layer relative to the moment the previous layer's last
    down-projection slice was stored."""
    import ctypes

    import velomind_hip as H
    from velomind_hip import llama as VL

    spec = E2E_MODELS["tinyllama_1.1b_int4"]

    class Cfg:
        pass

    cfg = Cfg()
    for k, v in spec["cfg"].items():
        setattr(cfg, k, v)
    lib = H.open_library()
    probe = np.zeros(1, np.uint64)
    if lib.vm_hip_decode_trace_read(probe.ctypes.data, 0) != 0:
        raise RuntimeError("--decode-trace needs libvmhip built with VELOMIND_DECODE_TRACE=1")
    w = VL.Weights(cfg)
    w.fill_synthetic(20240601, 0.02)
    prev = os.environ.get("VELOMIND_DECODE_PERSISTENT")
    os.environ["VELOMIND_DECODE_PERSISTENT"] = "1"
    try:
        sess = VL.Session(w, VL.ENGINE_RESIDENT, spec["quant"], spec["block"], max_seq=spec["prompt"] + tokens + 1)
    finally:
        if prev is None:
            del os.environ["VELOMIND_DECODE_PERSISTENT"]
        else:
            os.environ["VELOMIND_DECODE_PERSISTENT"] = prev
    if DECODE_PATHS[sess.decode_path()] != "persistent":
        raise RuntimeError("the persistent decode step does not cover TinyLlama here")
    prompt = np.random.default_rng(5).integers(0, cfg.vocab_size, spec["prompt"]).astype(np.int32)
    _, (_, dec_s, nd) = sess.generate(prompt, tokens)
    wgs, slots, events = 512, 34, 24
    buf = np.zeros(wgs * slots * events, np.uint64)
    H.check(lib.vm_hip_decode_trace_read(buf.ctypes.data, buf.nbytes))
    sess.close()
    w.close()
    t = buf.reshape(wgs, slots, events).astype(np.int64)
    L = cfg.num_layers
    live = t[:, 0, 0] > 0
    us = (t[live] - t[live, 0, 0].min()) / 100.0   # 100 MHz wall clock
    phases = [("qkv_stage", 0, 1), ("qkv_compute", 1, 2), ("qkv_store", 2, 3), ("attention", 4, 5),
              ("o_stage", 5, 6), ("o_compute", 6, 7), ("o_store", 7, 8), ("gate_up_stage", 8, 9),
              ("gate_up_compute", 9, 10), ("gate_up_store", 10, 11), ("down_stage", 11, 12),
              ("down_compute", 12, 13), ("down_store", 13, 14)]
    per_phase = {n: round(float(np.median(np.median(us[:, :L, b] - us[:, :L, a], axis=0))), 2) for n, a, b in phases}
    layer_us = np.median(us[:, 1:L, 0] - us[:, 0:L - 1, 0], axis=0)
    mid = L // 2
    z = us[:, mid - 1, 14].max()
    u = us[:, mid, :] - z
    att = u[:, 18] > -z   # workgroups that ran an attention item
    red = np.arange(us.shape[0] - 40, us.shape[0])
    chain = {"qkv_staged_median": float(np.median(u[:, 1])), "qkv_stored_max": float(u[:, 3].max()),
             "reduce_done_median": float(np.median(u[red, 16])),
             "attention_inputs_in_median": float(np.median(u[att, 17])),
             "attention_records_out_median": float(np.median(u[att, 18])),
             "o_staged_median": float(np.median(u[:, 6])), "o_stored_max": float(u[:, 8].max()),
             "gate_up_staged_median": float(np.median(u[:, 9])), "gate_up_stored_max": float(u[:, 11].max()),
             "down_staged_median": float(np.median(u[:, 12])), "down_stored_max": float(u[:, 14].max())}
    gu = us[:, mid, 10] - us[:, mid, 9]
    half = us.shape[0] // 2
    return {"model": "tinyllama_1.1b_int4", "prompt": spec["prompt"], "tokens": tokens,
            "decode_us_per_token": round(dec_s / nd * 1e6, 1), "workgroups": int(us.shape[0]),
            "layer_us_median": round(float(np.median(layer_us)), 2),
            "phase_us_median": per_phase,
            "layer_chain_us": {k: round(v, 2) for k, v in chain.items()},
            "gate_up_compute_us_by_workgroup_half": [round(float(np.median(gu[:half])), 2),
                                                     round(float(np.median(gu[half:])), 2)],
            "lm_head_us": round(float(np.median(us[:, L, 2] - us[:, L, 0])), 2),
            "argmax_us": round(float(us[0, L, 4] - np.median(us[:, L, 2])), 2)}


GEMM_K, GEMM_N = 2048, 5632
MFMA_F16_PEAK_TFLOPS = 2500.0


GEMV_TRACE_PHASES = ("entry_to_first_load", "first_load_to_staged", "chunk_reduce", "waves_summed",
                     "outputs_done")


def gemv_trace_report(H, stream, reps: int = 10) -> dict:
    """Phase timing of the decode GEMV (qmm_gemv.hip lists the events) from a
    library built with VELOMIND_GEMV_TRACE=1: for each TinyLlama-1.1B INT4
    decode shape and config 1's INT8 shape, one HIP graph of cold launches
    over a Rotation, replayed `reps` times; the last launch's timestamps as
    medians over its workgroups, the spread of their starts, the last
    workgroup's end, and the replay's time per launch (the rest of which is
    spent between kernels)."""
    lib = H.open_library()
    probe = np.zeros(1, np.uint64)
    if lib.vm_hip_gemv_trace_read(probe.ctypes.data, 0) != 0:
        raise RuntimeError("--gemv-trace needs libvmhip built with VELOMIND_GEMV_TRACE=1")
    wgs, events = 4096, 8

    def trace(launch_all, copies):
        launch_all()
        stream.synchronize()
        us = timed_replay(H, stream, launch_all, reps) * 1e3 / copies
        buf = np.zeros(wgs * events, np.uint64)
        H.check(lib.vm_hip_gemv_trace_read(buf.ctypes.data, buf.nbytes))
        t = buf.reshape(wgs, events)[:, :6].astype(np.int64)
        # workgroup 0 runs in every launch; slots past this grid hold older launches
        t = t[np.abs(t[:, 0] - t[0, 0]) < 2000]
        rel = (t - t[:, 0].min()) * 0.01   # us
        d = np.diff(rel, axis=1)
        end = float(rel[:, 5].max())
        return {"us_per_launch": round(us, 3), "workgroups": int(len(t)),
                "start_spread_us": round(float(rel[:, 0].max()), 2),
                "phases_us_median": {name: round(float(np.median(d[:, i])), 2)
                                     for i, name in enumerate(GEMV_TRACE_PHASES)},
                "last_done_us": round(end, 2), "between_kernels_us": round(us - end, 2)}

    out = {}
    wl = Workload(H, stream)
    for (k, n), (mp, ms) in sorted(wl.masters.items()):
        rot = Rotation(H, mp, ms, stream)

        def launch_all(rot=rot, k=k, n=n):
            for pa, sa in rot.addrs:
                H.qmm_f32(wl.x[k].addr, pa, sa, wl.out[n].addr, 1, k, n, H.QUANT_INT4, BLOCK, stream)

        out[f"int4_{k}x{n}"] = trace(launch_all, rot.copies)
        rot.close()
    k, n = CONFIG1_K, CONFIG1_N
    rng = np.random.default_rng(3)
    dw = H.DeviceBuffer.from_array((rng.standard_normal((k, n), dtype=np.float32) * np.float32(0.02)))
    p, s = H.DeviceBuffer(k * n), H.DeviceBuffer(n * 4)
    H.pack_int8(dw.addr, p.addr, s.addr, k, n)
    H.synchronize()
    dx, dc = H.DeviceBuffer.from_array(rng.standard_normal(k, dtype=np.float32)), H.DeviceBuffer(n * 4)
    rot = Rotation(H, p, s, stream)

    def launch_int8():
        for pa, sa in rot.addrs:
            H.qmm_f32(dx.addr, pa, sa, dc.addr, 1, k, n, H.QUANT_INT8, 0, stream)

    out[f"int8_{k}x{n}"] = trace(launch_int8, rot.copies)
    rot.close()
    for b in (dw, p, s, dx, dc):
        b.close()
    return out


def gemm_setup(H):
    """BASELINE config 3 operands: W [2048, 5632] N(0, 0.02) packed on the
    GPU as INT8 (per column) and INT4 (block 32); A [512, 2048] N(0, 1)."""
    rng = np.random.default_rng(11)
    w = (rng.standard_normal((GEMM_K, GEMM_N), dtype=np.float32) * np.float32(0.02)).astype(np.float32)
    dw = H.DeviceBuffer.from_array(w)
    packs = {}
    for qt in (H.QUANT_INT8, H.QUANT_INT4):
        if qt == H.QUANT_INT4:
            p = H.DeviceBuffer(GEMM_K // 2 * GEMM_N)
            s = H.DeviceBuffer(GEMM_K // BLOCK * GEMM_N * 4)
            H.pack_int4(dw.addr, p.addr, s.addr, GEMM_K, GEMM_N, BLOCK)
            packs[qt] = (p, s, BLOCK)
        else:
            p = H.DeviceBuffer(GEMM_K * GEMM_N)
            s = H.DeviceBuffer(GEMM_N * 4)
            H.pack_int8(dw.addr, p.addr, s.addr, GEMM_K, GEMM_N)
            packs[qt] = (p, s, 0)
    H.synchronize()
    dw.close()
    a = H.DeviceBuffer.from_array(rng.standard_normal((512, GEMM_K), dtype=np.float32))
    c = H.DeviceBuffer(512 * GEMM_N * 4)
    return packs, a, c


def gemm_bench(H, stream, reps: int = 5) -> dict:
    """Config 3, the MFMA path: M in {16, 128, 512} x INT8 / INT4, launched
    once per weight copy of a Rotation (>= 512 MB of copies, so that the
    weights stream from HBM, not from the Infinity Cache), as one HIP graph
    replayed `reps` times between events.  FLOPs 2*M*K*N; algorithmic bytes
    codes + scales + fp32 A + fp32 C."""
    packs, a, c = gemm_setup(H)
    rots = {qt: Rotation(H, p, s, stream) for qt, (p, s, _) in packs.items()}
    out = {}
    for m in (16, 128, 512):
        for qt in (H.QUANT_INT8, H.QUANT_INT4):
            blk = packs[qt][2]
            rot = rots[qt]

            def launch_all():
                for pa, sa in rot.addrs:
                    H.qmm_f32(a.addr, pa, sa, c.addr, m, GEMM_K, GEMM_N, qt, blk, stream)

            # an eager pass sizes the split-K and staging workspaces before capture
            launch_all()
            stream.synchronize()
            us = timed_replay(H, stream, launch_all, reps) * 1e3 / rot.copies
            flops = 2.0 * m * GEMM_K * GEMM_N
            codes = GEMM_K * GEMM_N if qt == H.QUANT_INT8 else GEMM_K // 2 * GEMM_N
            scales = GEMM_N * 4 if qt == H.QUANT_INT8 else GEMM_K // BLOCK * GEMM_N * 4
            nbytes = codes + scales + 4 * m * GEMM_K + 4 * m * GEMM_N
            tf = flops / (us * 1e-6) / 1e12
            out[f"M{m}_{'int8' if qt == H.QUANT_INT8 else 'int4'}"] = {
                "us": round(us, 2), "TFLOP_s": round(tf, 1), "frac_of_mfma_f16_peak": round(tf / MFMA_F16_PEAK_TFLOPS, 4),
                "GB_s": round(nbytes / (us * 1e-6) / 1e9, 1), "frac_of_hbm_peak": round(nbytes / (us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
                "rotation": f"{rot.copies} weight copies, {rot.bytes / 2**20:.0f} MiB"}
    for rot in rots.values():
        rot.close()
    for p, s, _ in packs.values():
        p.close()
        s.close()
    a.close()
    c.close()
    return out


CONFIG1_K, CONFIG1_N = 576, 1536


def config1_setup(H):
    """Config 1's operands: x [576] and W [576, 1536] ~ N(0, 0.02), W packed
    on the GPU (INT8 per column).  Returns x and the device buffers."""
    rng = np.random.default_rng(3)
    k, n = CONFIG1_K, CONFIG1_N
    w = (rng.standard_normal((k, n), dtype=np.float32) * np.float32(0.02)).astype(np.float32)
    x = rng.standard_normal(k, dtype=np.float32)
    dw = H.DeviceBuffer.from_array(w)
    p, s = H.DeviceBuffer(k * n), H.DeviceBuffer(n * 4)
    H.pack_int8(dw.addr, p.addr, s.addr, k, n)
    H.synchronize()
    dw.close()
    return x, p, s, H.DeviceBuffer.from_array(x), H.DeviceBuffer(n * 4)


def config1_bench(H, stream, reps: int = 10, cpu_seconds: float = 3.0) -> dict:
    """the INT8 per-column decode GEMV (M=1), K 576 x
    N 1536 (quantized_matmul.cpp:190-235's streaming decode shape).  W
    N(0, 0.02) packed on the GPU by vm_hip_pack_int8 (bit-exact with
    quant.cpp); launched once per weight copy of a Rotation (>= 512 MB) in
    one HIP graph replayed `reps` times.  The CPU leg is the oracle's
    restatement of decode_stream_int8_avx2 (quantized_matmul.cpp:146-188)
    on one pinned core, on the same codes (cache-resident: 0.9 MB)."""
    import oracle as O

    k, n = CONFIG1_K, CONFIG1_N
    x, p, s, dx, dc = config1_setup(H)
    rot = Rotation(H, p, s, stream)

    def launch_all():
        for pa, sa in rot.addrs:
            H.qmm_f32(dx.addr, pa, sa, dc.addr, 1, k, n, H.QUANT_INT8, 0, stream)

    launch_all()
    stream.synchronize()
    us = timed_replay(H, stream, launch_all, reps) * 1e3 / rot.copies
    nbytes = k * n + n * 4 + k * 4 + n * 4
    gbs = nbytes / (us * 1e-6) / 1e9
    out = {"shape_KxN": f"{k}x{n}", "us": round(us, 3), "algo_bytes_per_launch": nbytes, "GB_s": round(gbs, 1),
           "frac_of_hbm_peak": round(gbs / HBM_PEAK_GBS, 4),
           "rotation": f"{rot.copies} weight copies, {rot.bytes / 2**20:.0f} MiB"}
    rot.close()
    if cpu_seconds > 0:
        q = p.download(np.int8, (k, n))
        sc = s.download(np.float32, (n,))
        cpu = sorted(os.sched_getaffinity(0))[0]
        prev = os.sched_getaffinity(0)
        os.sched_setaffinity(0, {cpu})
        try:
            calls = 0
            t0 = time.perf_counter()
            while time.perf_counter() - t0 < cpu_seconds:
                for _ in range(50):
                    O.qmm_decode_int8(x, q, sc)
                calls += 50
            dt = time.perf_counter() - t0
        finally:
            os.sched_setaffinity(0, prev)
        out["cpu_baseline"] = {"value": round(nbytes * calls / dt / 1e9, 3), "unit": "GB/s", "cores": 1,
                               "kind": "port", "us_per_call": round(dt / calls * 1e6, 2),
                               "avx2_fma": O.has_avx2_fma(),
                               "sample": f"{calls} calls of the oracle's decode_stream_int8_avx2 restatement "
                                         f"(quantized_matmul.cpp:146-188) on core {cpu}, {dt:.1f} s, "
                                         "weights cache-resident"}
    for b in (p, s, dx, dc):
        b.close()
    return out


def fused_gemv_bench(H, stream, reps: int = 10) -> dict:
    """The graph engine's fused decode GEMVs (kernel.h FusedKind: NormQmm,
    QmmAdd, SwigluQmmAdd) beside the plain launches of the same products,
    at SmolLM2-360M INT8 shapes (M = 1): q|k|v and gate|up as sibling groups
    with and without the RMSNorm in their staging, o with and without the
    residual addend, down with and without the SwiGLU staging and addend.
    Each case is launched once per weight copy of Rotations walking >= 512 MB
    (cold HBM), as one HIP graph replayed `reps` times; microseconds per
    launch."""
    import ctypes

    lib = H.load()
    rng = np.random.default_rng(11)
    hid, kvd, inter = 960, 320, 2560

    def packed(k, n):
        w = (rng.standard_normal((k, n), dtype=np.float32) * np.float32(0.02)).astype(np.float32)
        dw = H.DeviceBuffer.from_array(w)
        p, sc = H.DeviceBuffer(k * n), H.DeviceBuffer(n * 4)
        H.pack_int8(dw.addr, p.addr, sc.addr, k, n)
        H.synchronize()
        dw.close()
        return p, sc

    vec = lambda n: H.DeviceBuffer.from_array(rng.standard_normal(n, dtype=np.float32))   # noqa: E731
    x, g, h = vec(inter), vec(inter), vec(inter)
    nw = H.DeviceBuffer.from_array((1 + 0.1 * rng.standard_normal(hid)).astype(np.float32))
    outs = [H.DeviceBuffer(inter * 4) for _ in range(3)]

    def rotations(shapes):
        mats = [packed(k, n) for k, n in shapes]
        copies = -(-ROTATION_BYTES // sum(k * n + n * 4 for k, n in shapes))
        rots = [Rotation(H, p, sc, stream, copies=copies) for p, sc in mats]
        for p, sc in mats:
            p.close()
            sc.close()
        return rots, copies

    def members(rots, shapes, i):
        arr = (H.QmmMember * len(rots))()
        for j, (r, (_, n)) in enumerate(zip(rots, shapes)):
            arr[j].codes, arr[j].scales = r.addrs[i]
            arr[j].c, arr[j].n = outs[j].addr, n
        return arr

    def time_case(rots, copies, launch_one) -> float:
        args = [launch_one(i) for i in range(copies)]   # ctypes arguments built outside the capture
        def launch_all():
            for f in args:
                f()
        launch_all()   # eager first: sizes any split-K workspace before the capture
        stream.synchronize()
        return timed_replay(H, stream, launch_all, reps) * 1e3 / copies

    eps = ctypes.c_float(1e-5)
    out = {}
    for name, shapes in (("q|k|v", ((hid, hid), (hid, kvd), (hid, kvd))), ("gate|up", ((hid, inter), (hid, inter)))):
        rots, copies = rotations(shapes)
        cnt = len(shapes)

        def plain(i, rots=rots, shapes=shapes, cnt=cnt):
            m = members(rots, shapes, i)
            return lambda: H.check(lib.vm_hip_qmm_group_f32(x.addr, 1, hid, m, cnt, H.QUANT_INT8, 0, stream.handle))

        def normed(i, rots=rots, shapes=shapes, cnt=cnt):
            m = members(rots, shapes, i)
            return lambda: H.check(lib.vm_hip_qmm_norm_group_f32(x.addr, nw.addr, eps, 1, hid, m, cnt, H.QUANT_INT8,
                                                                 0, stream.handle))

        a, b = time_case(rots, copies, plain), time_case(rots, copies, normed)
        out[name] = {"KxN": f"{hid}x{'|'.join(str(n) for _, n in shapes)}", "plain_group_us": round(a, 3),
                     "with_rmsnorm_us": round(b, 3), "copies": copies}
        for r in rots:
            r.close()
    for name, (k, n), fused, what in (("o", (hid, hid), "qmm_add", "with_addend_us"),
                                      ("down", (inter, hid), "swiglu_add", "with_swiglu_and_addend_us")):
        rots, copies = rotations(((k, n),))
        r = rots[0]

        def plain(i, k=k, n=n, r=r):
            pa, sa = r.addrs[i]
            return lambda: H.check(lib.vm_hip_qmm_f32(x.addr, pa, sa, outs[0].addr, 1, k, n, H.QUANT_INT8, 0,
                                                      stream.handle))

        def add(i, k=k, n=n, r=r):
            pa, sa = r.addrs[i]
            return lambda: H.check(lib.vm_hip_qmm_add_f32(x.addr, pa, sa, h.addr, outs[0].addr, 1, k, n,
                                                          H.QUANT_INT8, 0, stream.handle))

        def swiglu(i, k=k, n=n, r=r):
            pa, sa = r.addrs[i]
            return lambda: H.check(lib.vm_hip_qmm_swiglu_add_f32(g.addr, x.addr, pa, sa, h.addr, outs[0].addr, 1, k,
                                                                 n, H.QUANT_INT8, 0, stream.handle))

        a = time_case(rots, copies, plain)
        b = time_case(rots, copies, add if fused == "qmm_add" else swiglu)
        out[name] = {"KxN": f"{k}x{n}", "plain_us": round(a, 3), what: round(b, 3), "copies": copies}
        r.close()
    for buf in (x, g, h, nw, *outs):
        buf.close()
    return out


LARGE_SHAPES = ((8192, 28672), (28672, 8192), (8192, 128256))


def large_gemv_bench(H, stream, reps: int = 5) -> dict:
    """Decode GEMVs (M=1, INT4 block 32) at 70B-class shapes, where a launch
    moves 150-660 MB and latency no longer dominates: Llama-3-70B-shaped
    gate/up (8192 x 28672), down (28672 x 8192) and lm_head (8192 x 128256).
    Weights N(0, 0.02) drawn and packed on the GPU; enough copies per HIP
    graph (>= 700 MB) that replays read cold HBM, not the 256 MB Infinity
    Cache.  Same kernel and config rule as the sweep."""
    lib = H.open_library()
    rng = np.random.default_rng(5)
    out = {}
    for k, n in LARGE_SHAPES:
        x = H.DeviceBuffer.from_array(rng.standard_normal(k, dtype=np.float32))
        c = H.DeviceBuffer(n * 4)
        w = H.DeviceBuffer(k * n * 4)
        H.check(lib.vm_hip_fill_normal_f32(w.ptr, k * n, 77, 0.0, 0.02, None))
        pb, sb = k // 2 * n, k // BLOCK * n * 4
        copies = max(2, -(-700_000_000 // (pb + sb)))
        packs = []
        for i in range(copies):
            p, s = H.DeviceBuffer(pb), H.DeviceBuffer(sb)
            if i == 0:
                H.pack_int4(w.addr, p.addr, s.addr, k, n, BLOCK)
            else:
                H.check(lib.vm_hip_memcpy_d2d(p.ptr, packs[0][0].ptr, pb, None))
                H.check(lib.vm_hip_memcpy_d2d(s.ptr, packs[0][1].ptr, sb, None))
            packs.append((p, s))
        H.synchronize()
        w.close()
        for p, s in packs:
            H.qmm_f32(x.addr, p.addr, s.addr, c.addr, 1, k, n, H.QUANT_INT4, BLOCK, stream)
        stream.synchronize()
        g = H.Graph(stream)
        g.begin()
        for p, s in packs:
            H.qmm_f32(x.addr, p.addr, s.addr, c.addr, 1, k, n, H.QUANT_INT4, BLOCK, stream)
        g.end()
        g.launch()
        stream.synchronize()
        e0, e1 = H.Event(), H.Event()
        e0.record(stream.handle)
        for _ in range(reps):
            g.launch()
        e1.record(stream.handle)
        e1.synchronize()
        g.close()
        us = e0.elapsed_ms(e1) * 1e3 / (reps * copies)
        nbytes = algo_bytes(k, n)
        gbs = nbytes / (us * 1e-6) / 1e9
        out[f"{k}x{n}"] = {"us": round(us, 2), "algo_bytes": nbytes, "GB_s": round(gbs, 1),
                           "frac_of_hbm_peak": round(gbs / HBM_PEAK_GBS, 4), "copies": copies}
        for p, s in packs:
            p.close()
            s.close()
        x.close()
        c.close()
    return out


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--no-graph", action="store_true", help="launch eagerly instead of replaying a HIP graph")
    ap.add_argument("--shape-reps", type=int, default=20, help="replays per shape for per-launch durations")
    ap.add_argument("--cpu-seconds", type=float, default=12.0, help="bounded CPU-baseline sample (0 = skip)")
    ap.add_argument("--only-shape", default="", help="KxN: launch only this shape's GEMVs (profiling passes)")
    ap.add_argument("--no-e2e", action="store_true", help="skip the end-to-end decode legs (configs 4 and 5)")
    ap.add_argument("--e2e-only", action="store_true",
                    help="only the end-to-end legs, printed as one JSON line (profiling passes; with --no-graph "
                         "the decode steps launch eagerly so that rocprofv3 can trace them)")
    ap.add_argument("--decode-persistent", action="store_true",
                    help="with --e2e-only: decode with the one-launch step (vm_hip_decode_step)")
    ap.add_argument("--e2e-model", default="", choices=[""] + list(E2E_MODELS),
                    help="with --e2e-only: only this model")
    ap.add_argument("--e2e-steps", type=int, default=0,
                    help="with --e2e-only: decode this many tokens instead of the config's (short profiling runs)")
    ap.add_argument("--e2e-layers", default="",
                    help="with --e2e-only and --e2e-model: comma-separated layer counts to run instead of the "
                         "config's (per-layer decode time with the weights resident in the 256 MB Infinity Cache "
                         "at few layers, streamed from HBM at many)")
    ap.add_argument("--fused-gemv", action="store_true",
                    help="only the graph engine's fused decode GEMVs beside the plain ones (SmolLM2 INT8 shapes)")
    ap.add_argument("--graph-engine", action="store_true",
                    help="only the drop-in graph-engine decode of config 4 (both attention forms)")
    ap.add_argument("--gemv-trace", action="store_true",
                    help="phase timestamps of the decode GEMV per shape (library built with VELOMIND_GEMV_TRACE=1)")
    ap.add_argument("--decode-trace", action="store_true",
                    help="only the one-launch decode step's phase timestamps (library built with "
                         "VELOMIND_DECODE_TRACE=1), printed as one JSON line")
    ap.add_argument("--no-gemm", action="store_true", help="skip the prefill GEMM leg (config 3)")
    ap.add_argument("--no-large", action="store_true", help="skip the 70B-class decode GEMV leg")
    ap.add_argument("--gemm-only", action="store_true", help="only the prefill GEMM leg, printed as one JSON line")
    ap.add_argument("--gemm-profile", default="",
                    help="M,QT,REPS: only REPS eager launches of one config-3 GEMM, each on the next weight copy "
                         "of a >= 512 MB rotation (rocprofv3 counter passes)")
    ap.add_argument("--config1-profile", type=int, default=0,
                    help="REPS: only REPS eager launches of config 1's INT8 GEMV, each on the next weight copy "
                         "of a >= 512 MB rotation (rocprofv3 counter passes)")
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="only run ten 64 MiB device-to-device copies (rocprofv3 counter calibration)")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py: this build measures one GPU; --gpus must be 1 (no multi-GPU path is built)",
              file=sys.stderr)
        return 2

    import velomind_hip as H

    H.load()
    stream = H.Stream()
    if args.calibrate_copy:
        src, dst = H.DeviceBuffer(64 << 20), H.DeviceBuffer(64 << 20)
        lib = H.open_library()
        for _ in range(10):
            H.check(lib.vm_hip_memcpy_d2d(dst.ptr, src.ptr, 64 << 20, stream.handle))
        stream.synchronize()
        log("bench: calibration copies done (10 x 64 MiB)")
        return 0
    if args.gemm_profile:
        m, qt, reps = (int(v) for v in args.gemm_profile.split(","))
        packs, a, c = gemm_setup(H)
        p, s, blk = packs[qt]
        rot = Rotation(H, p, s, stream)
        for i in range(reps):
            pa, sa = rot.addrs[i % rot.copies]
            H.qmm_f32(a.addr, pa, sa, c.addr, m, GEMM_K, GEMM_N, qt, blk, stream)
        stream.synchronize()
        log(f"bench: {reps} GEMM launches M={m} quant_type={qt} done, walking {rot.copies} weight copies")
        return 0
    if args.config1_profile:
        _, p, s, dx, dc = config1_setup(H)
        rot = Rotation(H, p, s, stream)
        for i in range(args.config1_profile):
            pa, sa = rot.addrs[i % rot.copies]
            H.qmm_f32(dx.addr, pa, sa, dc.addr, 1, CONFIG1_K, CONFIG1_N, H.QUANT_INT8, 0, stream)
        stream.synchronize()
        log(f"bench: {args.config1_profile} config-1 GEMV launches done, walking {rot.copies} weight copies")
        return 0
    if args.decode_trace:
        print(json.dumps({"metric": METRIC, "decode_trace": decode_trace_report()}), flush=True)
        return 0
    if args.gemv_trace:
        print(json.dumps({"metric": METRIC, "gemv_trace": gemv_trace_report(H, stream)}), flush=True)
        return 0
    if args.gemm_only:
        print(json.dumps({"metric": METRIC, "gemm": gemm_bench(H, stream)}), flush=True)
        return 0
    if args.e2e_only and args.e2e_layers:
        if not args.e2e_model:
            log("bench: --e2e-layers needs --e2e-model")
            return 2
        base = E2E_MODELS[args.e2e_model]
        rows = []
        for layers in (int(v) for v in args.e2e_layers.split(",")):
            name = f"{args.e2e_model}_{layers}_layers"
            E2E_MODELS[name] = dict(base, cfg=dict(base["cfg"], num_layers=layers))
            wb = decode_weight_bytes(E2E_MODELS[name]["cfg"], base["quant"], base["block"])
            for persistent in (False, True):
                r = e2e_bench(name, persistent=persistent, steps=args.e2e_steps or 48)
                rows.append({"layers": layers, "decode_path": r["decode_path"], "weight_MB_per_token": round(wb / 1e6, 1),
                             "decode_us_per_token": r["decode_us_per_token"],
                             "us_per_layer": round(r["decode_us_per_token"] / layers, 2)})
                log(f"bench: {name} {r['decode_path']}: {r['decode_us_per_token']} us/token")
        print(json.dumps({"metric": METRIC, "e2e_layers": rows}), flush=True)
        return 0
    if args.fused_gemv:
        print(json.dumps({"metric": METRIC, "fused_gemv": fused_gemv_bench(H, stream)}), flush=True)
        return 0
    if args.graph_engine:
        out = {}
        for name, steps in GRAPH_ENGINE_E2E.items():
            for fa in (False, True):
                out[f"{name}{'_fused_attention' if fa else ''}"] = e2e_bench(name, graph_engine=True, steps=steps,
                                                                              fused_attention=fa)
        print(json.dumps({"metric": METRIC, "graph_engine": out}), flush=True)
        return 0
    if args.e2e_only:
        e2e = {}
        for name in [args.e2e_model] if args.e2e_model else E2E_MODELS:
            log(f"bench: end-to-end {name}")
            e2e[name] = e2e_bench(name, use_graph=not args.no_graph, persistent=args.decode_persistent,
                                  steps=args.e2e_steps)
            log(f"bench: {name}: prefill {e2e[name]['prefill_tokens_per_s']} tok/s, "
                f"decode {e2e[name]['decode_tokens_per_s']} tok/s ({e2e[name]['decode_path']})")
        print(json.dumps({"metric": METRIC, "e2e": e2e}), flush=True)
        return 0
    log("bench: packing weights on the GPU")
    wl = Workload(H, stream)
    if args.only_shape:
        k_only, n_only = (int(v) for v in args.only_shape.split("x"))
        wl.calls = [c for c in wl.calls if (c[1], c[2]) == (k_only, n_only)]
        if not wl.calls:
            log(f"bench: no GEMV of shape {args.only_shape} in the step")
            return 2
        wl.bytes_per_step = sum(algo_bytes(k, n) for _, k, n, _, _ in wl.calls)
    log(f"bench: {len(wl.calls)} GEMVs per step, {wl.bytes_per_step / 1e6:.1f} MB per step")

    # eager warm-up sizes the split-K workspace before any capture
    for _ in range(2):
        wl.launch_step()
    stream.synchronize()

    graph = None
    if not args.no_graph:
        graph = H.Graph(stream)
        graph.begin()
        wl.launch_step()
        graph.end()

    def run_step():
        if graph is not None:
            graph.launch()
        else:
            wl.launch_step()

    for _ in range(args.warmup):
        run_step()
    stream.synchronize()
    H.synchronize()

    e0, e1 = H.Event(), H.Event()
    wall0 = time.perf_counter()
    e0.record(stream.handle)
    for _ in range(args.steps):
        run_step()
    e1.record(stream.handle)
    e1.synchronize()
    H.synchronize()
    wall = time.perf_counter() - wall0
    ms_total = e0.elapsed_ms(e1)
    ms_per_step = ms_total / args.steps
    value = wl.bytes_per_step / (ms_per_step * 1e-3) / 1e9
    log(f"bench: {ms_per_step * 1e3:.1f} us/step, {value:.1f} GB/s (wall {wall:.2f} s)")

    # Per-step distribution (median and P95, as the reference's
    # benchmarks/stats_helper.h:19-40 reports): steps after the timed
    # region, each between its own pair of events.
    ev = [H.Event() for _ in range(min(args.steps, 100) + 1)]
    ev[0].record(stream.handle)
    for i in range(1, len(ev)):
        run_step()
        ev[i].record(stream.handle)
    ev[-1].synchronize()
    per_step = np.array([ev[i - 1].elapsed_ms(ev[i]) for i in range(1, len(ev))])
    step_stats = {"samples": int(per_step.size), "median_ms": round(float(np.median(per_step)), 5),
                  "p95_ms": round(float(np.percentile(per_step, 95)), 5),
                  "min_ms": round(float(per_step.min()), 5), "max_ms": round(float(per_step.max()), 5)}

    # The same sweep with sibling GEMVs grouped (one launch per q | k | v
    # and per gate | up), as the drop-in graph path runs them on HIP.
    grouped = None
    if not args.only_shape:
        groups = wl.grouped_calls()
        wl.launch_grouped_step(groups)
        stream.synchronize()
        gg = H.Graph(stream)
        gg.begin()
        wl.launch_grouped_step(groups)
        gg.end()
        for _ in range(args.warmup):
            gg.launch()
        stream.synchronize()
        g0, g1 = H.Event(), H.Event()
        g0.record(stream.handle)
        for _ in range(args.steps):
            gg.launch()
        g1.record(stream.handle)
        g1.synchronize()
        gms = g0.elapsed_ms(g1) / args.steps
        gg.close()
        grouped = {"launches_per_step": len(groups), "ms_per_step": round(gms, 5),
                   "GB_s": round(wl.bytes_per_step / (gms * 1e-3) / 1e9, 1),
                   "pct_of_hbm_peak": round(100.0 * wl.bytes_per_step / (gms * 1e-3) / 1e9 / HBM_PEAK_GBS, 2),
                   "gemv_tokens_per_s": round(1e3 / gms, 1),
                   "grouping": "per layer q|k|v (2048 x 2560) and gate|up (2048 x 11264) as one "
                               "vm_hip_qmm_group_f32 launch each; o, down, lm_head alone",
                   "algo_bytes_per_step": wl.bytes_per_step}
        log(f"bench: grouped sweep {gms * 1e3:.1f} us/step, {grouped['GB_s']} GB/s")

    durs = per_shape_durations(H, wl, args.shape_reps, graph is not None)
    per_shape = {}
    for (k, n), (ms, count, copies, rbytes) in durs.items():
        b = algo_bytes(k, n)
        per_shape[f"{k}x{n}"] = {"launches_per_step": count, "avg_launch_us": round(ms * 1e3, 3),
                                 "algo_bytes_per_launch": b, "GB_s": round(b / (ms * 1e-3) / 1e9, 1),
                                 "us_per_step": round(ms * 1e3 * count, 1),
                                 "rotation": f"{copies} weight copies, {rbytes / 2**20:.0f} MiB"}
    # The roofline is reported for the dominant kernel: the shape whose
    # launches take the most time per step.
    (dk, dn), (dms, dcount, _, _) = max(durs.items(), key=lambda kv: kv[1][0] * kv[1][1])
    dbytes = algo_bytes(dk, dn)
    achieved = dbytes / (dms * 1e-3) / 1e9
    launches = len(wl.calls)
    traffic, traffic_src = measured_traffic(f"{dk}x{dn}")

    e2e = None
    if not args.no_e2e and not args.only_shape:
        e2e = {}
        for name in E2E_MODELS:
            log(f"bench: end-to-end {name}")
            e2e[name] = e2e_bench(name)
            pers = e2e_bench(name, persistent=True)
            e2e[name]["persistent_step"] = {k: pers[k] for k in ("decode_tokens_per_s", "decode_us_per_token")}
            log(f"bench: {name}: prefill {e2e[name]['prefill_tokens_per_s']} tok/s, "
                f"decode {e2e[name]['decode_tokens_per_s']} tok/s ({e2e[name]['decode_path']}), "
                f"persistent step {pers['decode_tokens_per_s']} tok/s")
            if name in GRAPH_ENGINE_E2E:
                keys = ("prefill_tokens_per_s", "prefill_ms", "decode_tokens", "decode_tokens_per_s",
                        "decode_us_per_token", "host_ms_per_step", "bound", "attention", "engine")
                ge = e2e_bench(name, graph_engine=True, steps=GRAPH_ENGINE_E2E[name])
                gf = e2e_bench(name, graph_engine=True, steps=GRAPH_ENGINE_E2E[name], fused_attention=True)
                e2e[name]["graph_engine"] = {k: ge[k] for k in keys}
                e2e[name]["graph_engine"]["fused_attention"] = {k: gf[k] for k in keys if k != "engine"}
                log(f"bench: {name} graph engine: prefill {ge['prefill_tokens_per_s']} tok/s, "
                    f"decode {ge['decode_tokens_per_s']} tok/s; use_fused_attention: "
                    f"decode {gf['decode_tokens_per_s']} tok/s")

    gemm = None
    if not args.no_gemm and not args.only_shape:
        log("bench: prefill GEMM (config 3)")
        gemm = gemm_bench(H, stream)

    config1 = None
    if not args.only_shape:
        log("bench: INT8 decode GEMV (config 1)")
        config1 = config1_bench(H, stream, cpu_seconds=3.0 if args.cpu_seconds > 0 else 0.0)

    large = None
    if not args.no_large and not args.only_shape:
        log("bench: 70B-class decode GEMVs")
        large = large_gemv_bench(H, stream)

    cpu = None
    if args.cpu_seconds > 0:
        log("bench: timing CPU baseline")
        cpu = cpu_baseline(args.cpu_seconds)

    result = {
        "metric": METRIC,
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic",
        "config": {
            "workload": "tinyllama_1.1b_int4_decode_gemv_sweep",
            "gemvs_per_step": launches,
            "layers": LAYERS,
            "shapes_KxN": [f"{k}x{n}" for _, k, n in LAYER_SHAPES] + [f"{LM_HEAD[1]}x{LM_HEAD[2]}"],
            "weights": "int4 block 32, quant.cpp layout, packed on GPU from N(0,0.02)",
            "activations": "fp32 N(0,1), M=1",
            "bytes_per_step": wl.bytes_per_step,
            "launch": "eager" if graph is None else "hip_graph",
        },
        "gemv_tokens_per_s": round(1e3 / ms_per_step, 1),
        "pct_of_hbm_peak": round(100.0 * value / HBM_PEAK_GBS, 2),
        "roofline": {
            "bound": "hbm",
            "achieved": round(achieved, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4),
            "traffic": traffic,
            "traffic_source": traffic_src,
            "kernel": f"qmm_gemv_kernel, INT4 K={dk} N={dn} (M=1), {dcount} launches per step",
            "avg_launch_us": round(dms * 1e3, 3),
            "algo_bytes_per_launch": dbytes,
        },
        "step_stats": step_stats,
        "grouped_sweep": grouped,
        "per_shape": per_shape,
        "e2e": e2e,
        "config1_int8_gemv": config1,
        "gemm": gemm,
        "gemv_large": large,
        "cpu_baseline": cpu,
    }
    print(json.dumps(result), flush=True)
    if graph is not None:
        graph.close()
    return 0


if __name__ == "__main__":
    sys.exit(main())
