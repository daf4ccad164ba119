"""Throughput of the per-token Mamba-130M step on one MI355X through libredukt_gpu.so.

Default workload: Mamba-130M with int8 weight-only quantisation (per-output-row f32
scales on in_proj, x_proj, dt_proj, out_proj and the tied head; f32 activations and
state), 128 lockstep streams with independent Zipf(1.1) token ids, every stream's state
reset at the 4096-token boundary (placed inside the timed region).  A step is one token
for each of the 128 streams.  Inputs (weights, token ids, slots) are resident in HBM
before timing starts; logits stay on the device.

Prints one JSON line.  `value` is that workload's tokens/s.  `grid` adds the rest of the
metric, Mamba-130M at 1, 32 and 128 streams with F32 and int8 weights: device tok/s
(logits left on the device) and FFI tok/s (synchronous forward_batch into host memory).
`roofline` covers the dominant kernel of the default workload (HIP events on the
library's stream around each of its launches inside full steps, in a probe pass after
the timed region); `configs` adds the other workloads' device rates (F32 probabilities
at 128 streams, RWKV-7 0.1B at 64 streams); `cpu_baseline` times the CPU oracle (a C
restatement of the reference CPU path) on the host cores for a bounded sample of the
same workload, with all of one GPU's share of the cores and with one.
"""
from __future__ import annotations

import argparse
import ctypes
import json
import os
import sys
import tempfile
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

from redukt_amd import ffi, hip, rbin, rwkv, synth  # noqa: E402

METRIC = "Mamba-130M tok/s at batch 1/32/128 (F32 & Q8); % of HBM roofline"
HBM_PEAK_GBS = 8000.0
RESET_PERIOD = 4096
PROFILES = {"f32": 0, "q8": 1, "q8row": 2, "q8row-all": 6, "q8-all": 5,
            "f32-gemv": 16, "q8row-gemv": 18, "q8row-all-gemv": 22, "q8row-w8a8": 34,
            "f32-ref": 64, "q8-ref": 65, "q8row-all-ref": 70, "f32-ref-fma": 192, "q8-ref-fma": 193}


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def weight_bytes(dims: rbin.MambaDims, profile: int) -> dict:
    """HBM bytes of each projection as stored on the device (weights + scales)."""
    d, di, dr, xr, V = dims.d_model, dims.d_inner, dims.dt_rank, dims.xr, dims.vocab
    q = profile & 3
    small_q = q and (profile & 4)

    def mat(rows, cols, quant):
        if not quant:
            return rows * cols * 4
        g = cols if q == 2 else (64 if cols % 64 == 0 else cols)
        return rows * cols + rows * (cols // g) * 4

    return {"in_proj": mat(2 * di, d, q), "x_proj": mat(xr, di, small_q), "dt_proj": mat(di, dr, small_q),
            "out_proj": mat(d, di, q), "head": mat(V, d, q)}


def algorithmic_bytes(dims: rbin.MambaDims, profile: int, n: int) -> dict:
    """Compulsory HBM bytes of one launch of each kernel class at n streams: weights once,
    every activation and state element read or written once.  x_proj's output counts once
    (written by mix_in, read by scan), not the split-K partials the kernels pass."""
    d, di, xr, V, dc = dims.d_model, dims.d_inner, dims.xr, dims.vocab, dims.d_conv
    w = weight_bytes(dims, profile)
    f = 4
    emb_row = d * f if profile & 3 == 0 else d + (4 if profile & 3 == 2 else d // 64 * f)
    return {
        "embed": n * (emb_row + d * f),
        # norm weights, in_proj, x_proj; x in; conv state in+out; conv w/b; u, z, x_proj output out
        "mix_in": d * f + w["in_proj"] + w["x_proj"] + n * d * f + n * 2 * di * (dc - 1) * f + di * (dc + 1) * f
        + n * 2 * di * f + n * xr * f,
        # x_proj output in; dt_proj, dt_b, exp(A_log), D; u, z in; ssm state in+out; gated out
        # (the f32 value: the kernels' bf16 limb encoding of it is not algorithmic)
        "scan": n * xr * f + w["dt_proj"] + di * f + di * 16 * f + di * f + n * 2 * di * f
        + n * 2 * di * 16 * f + n * di * f,
        # out_proj; gated in (f32); residual in+out
        "mix_out": w["out_proj"] + n * di * f + 2 * n * d * f,
        # final norm, head, x in, logits out
        "head": d * f + w["head"] + n * d * f + n * V * f,
        "softmax": 2 * n * V * f,
    }


def step_bytes(dims: rbin.MambaDims, profile: int, n: int) -> int:
    """Whole-step compulsory HBM bytes: weights once, state read+write, embedding rows,
    logits write (the B(N) of the workload description)."""
    wb = weight_bytes(dims, profile)
    L, d, di, dc = dims.n_layer, dims.d_model, dims.d_inner, dims.d_conv
    # every layer's four projections, then the head (tied: the embedding) once
    w = L * (wb["in_proj"] + wb["x_proj"] + wb["dt_proj"] + wb["out_proj"]) + wb["head"]
    # per layer: norm_w, conv_w, conv_b, dt_b, exp(A_log), D; then norm_f
    small = L * (d + di * dc + di + di + 16 * di + di) * 4 + d * 4
    state = 2 * L * di * ((dc - 1) + 16) * 4
    return w + small + n * (state + dims.vocab * 4 + d * 4)


def launches_per_step(dims, name: str, mamba: bool, profile: int) -> int:
    L = dims.n_layer
    if mamba:
        return L if name in ("mix_in", "scan", "mix_out") else 1
    if profile & ffi.PROFILE_EXACT:                       # r/k/v, two LoRA stages, o, FFN key, value
        return {"shift": 2 * L + 1, "proj": 6 * L, "wkv": L}.get(name, 1)
    if profile & ffi.PROFILE_W8A8:                        # + ln_out, staged as int8 for the head;
        return {"shift": 2 * L + 1, "proj": 6 * L, "wkv": L}.get(name, 1)   # proj: five products + k_quant_a8
    ws = (profile & 3) == 2 and dims.d_model <= 768       # the weights-stationary head needs ln_out staged
    return {"shift": 2 * L + (1 if ws else 0), "proj": 5 * L, "wkv": L}.get(name, 1)


def rwkv_weight_bytes(dims, profile: int) -> dict:
    d, f, V = dims.d_model, dims.d_ffn, dims.vocab
    q = profile & 3

    def mat(rows, cols):
        if not q:
            return rows * cols * 4
        g = cols if q == 2 else (64 if cols % 64 == 0 else cols)
        return rows * cols + rows * (cols // g) * 4

    ranks = dims.lora_w + dims.lora_a + dims.lora_v + dims.lora_g
    per_layer = 4 * mat(d, d) + mat(f, d) + mat(d, f) + 2 * d * ranks * 4
    return {"proj": dims.n_layer * per_layer, "head": mat(V, d), "emb_row": d * 4}


def rwkv_algorithmic_bytes(dims, profile: int, n: int) -> dict:
    """Compulsory HBM bytes per launch of each RWKV-7 kernel class at n streams (the step's
    bytes of that class over its launches): weights once, activations and state read or
    written once at f32."""
    d, f, V, L, H = dims.d_model, dims.d_ffn, dims.vocab, dims.n_layer, dims.n_head
    w = rwkv_weight_bytes(dims, profile)
    R = dims.lora_w + dims.lora_a + dims.lora_v + dims.lora_g
    if profile & ffi.PROFILE_W8A8:
        # int8 activations out of the LayerNorms (1 byte), f32 elsewhere.  Per stream and
        # layer: r/k/v + LoRA 1 (3d int8 + 4d f32 in, 3d + R out), LoRA 2 (R in, 4d out), output
        # (d f32 in, x read and written), FFN key (d int8 in, f out), FFN value (f in, x read
        # and written)
        proj = w["proj"] + n * L * (3 * d + 4 * (4 * d + 3 * d + R) + 4 * (R + 4 * d) + 4 * d + 4 * 2 * d + d
                                    + 4 * f + 4 * f + 4 * 2 * d)
        wkv = L * (n * (2 * H * 64 * 64 * 4 + 4 * (3 * d + 4 * d + 2 * d) + 4 * d) + 9 * d * 4)
        shift = n * (L * (4 * 3 * d + 3 * d + 4 * 4 * d) + L * (4 * 3 * d + d) + 4 * d + d)
        return {"embed": n * (w["emb_row"] + d * 4), "proj": proj // (5 * L), "wkv": wkv // L,
                "shift": shift // (2 * L + 1), "head": w["head"] + n * d + n * V * 4, "softmax": 2 * n * V * 4}
    ws = (profile & 3) == 2 and d <= 768
    proj = w["proj"] + n * L * 4 * (7 * d + 3 * d + 2 * R + 4 * d + 3 * d + d + f + f + 2 * d)
    wkv = L * (n * (2 * H * 64 * 64 * 4 + 8 * d * 4 + 2 * d * 4) + 9 * d * 4)
    shift = n * d * 4 * (L * (1 + 2 + 6) + L * (1 + 2 + 1) + (2 if ws else 0))
    return {"embed": n * (w["emb_row"] + d * 4), "proj": proj // (5 * L), "wkv": wkv // L,
            "shift": shift // (2 * L + (1 if ws else 0)), "head": w["head"] + n * d * 4 + n * V * 4,
            "softmax": 2 * n * V * 4}


def rwkv_step_bytes(dims, profile: int, n: int) -> int:
    d, V, L, H = dims.d_model, dims.vocab, dims.n_layer, dims.n_head
    w = rwkv_weight_bytes(dims, profile)
    state = L * (2 * d + H * 64 * 64) * 4 * 2
    return w["proj"] + w["head"] + L * 16 * d * 4 + n * (state + V * 4 + d * 4)


def ensure_rwkv(path: str) -> str:
    if not (os.path.isfile(path) and os.path.getsize(path) == rwkv.file_bytes(rwkv.RWKV7_0_1B)):
        log(f"writing synthetic RWKV-7 0.1B weights to {path}")
        rwkv.write_synthetic(path, rwkv.RWKV7_0_1B, seed=0)
    return path


def ensure_model(path: str) -> str:
    dims = rbin.MAMBA_130M
    expect = 44 + 4 * sum(int(np.prod(s)) for _, s in rbin.tensor_order(dims))
    if not (os.path.isfile(path) and os.path.getsize(path) == expect):
        log(f"writing synthetic Mamba-130M weights to {path}")
        synth.write_synthetic_mamba(path, dims, seed=0)
    return path


def cpu_info() -> dict:
    model = "unknown"
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    try:
        avail = len(os.sched_getaffinity(0))
    except AttributeError:
        avail = os.cpu_count() or 1
    return {"nproc": os.cpu_count() or 1, "affinity": avail, "model": model}


def cpu_baseline(path: str, profile: int, n: int, tokens: np.ndarray, budget_s: float, mamba: bool = True,
                 probs: bool = False) -> dict:
    """The oracle stepping the same workload on the host cores: first with one GPU's share
    of them (16, or fewer if the process may use fewer), then one step on one thread."""
    from oracle import oracle as O   # the CPU restatement; test/baseline infrastructure only

    info = cpu_info()
    threads = max(1, min(info["affinity"], 16))
    O.set_threads(threads)
    m = O.MambaOracle(path, profile, cap=n) if mamba else O.RwkvOracle(path, profile, cap=n)
    slots = list(range(n))

    def fwd(t: int) -> None:
        logits = m.forward(slots, [int(x) for x in tokens[t % len(tokens)]])
        if probs:                                           # softmax_into per stream, on the host
            for r in logits:
                O.softmax(r)

    fwd(0)                                                  # warm-up step
    t0 = time.perf_counter()
    fwd(1)
    one = time.perf_counter() - t0
    steps = max(1, int(budget_s / max(one, 1e-6)))
    t0 = time.perf_counter()
    for t in range(steps):
        fwd(2 + t)
    dt = time.perf_counter() - t0
    # one thread, one step (the caches are warm from the steps above)
    O.set_threads(1)
    t1 = time.perf_counter()
    fwd(2 + steps)
    dt1 = time.perf_counter() - t1
    O.set_threads(threads)
    m.close()
    return {"value": round(n * steps / dt, 2), "unit": "tok/s", "cores": threads, "kind": "port",
            "sample": f"CPU oracle{' + softmax per stream' if probs else ''}, same weights and profile, "
                      f"{n} lockstep streams x {steps} steps ({dt:.1f} s) on {threads} threads after one "
                      f"warm-up step; then 1 step on 1 thread ({dt1:.1f} s)",
            "value_1_thread": round(n / dt1, 2), "nproc": info["nproc"], "affinity": info["affinity"],
            "cpu_model": info["model"]}


class Workload:
    """One backend instance stepping n lockstep streams on device-resident inputs."""

    def __init__(self, be, n: int, vocab: int, tokens: np.ndarray, probs: bool = False):
        self.be, self.n, self.vocab, self.probs = be, n, vocab, probs
        self.tokens = tokens
        be.batch_init(n)
        self.stream = be.stream()
        self.d_tokens = hip.DeviceBuffer.from_array(tokens)
        self.d_slots = hip.DeviceBuffer.from_array(np.arange(n, dtype=np.uint32))
        self.d_out = hip.DeviceBuffer(n * vocab * 4)
        self.since = 0

    def step(self, t: int) -> None:
        if self.since >= RESET_PERIOD:                 # PluginState::tick for every stream
            self.be.batch_reset(None)
            self.since = 0
        self.since += 1
        t %= len(self.tokens)
        self.be.forward_batch_device(self.n, self.d_slots.ptr, self.d_tokens.ptr + t * self.n * 4, self.d_out.ptr,
                                     probs=self.probs)

    def timed(self, W: int, K: int, reset_at: int = -1):
        """W untimed steps, then K steps between two HIP events on the library's stream.
        With reset_at >= 0 the 4096-token boundary falls on timed step reset_at."""
        self.since = RESET_PERIOD - W - reset_at if reset_at >= 0 else 0
        for t in range(W):
            self.step(t)
        assert self.be.device_status() == ffi.BackendResult.OK
        e0, e1 = hip.Event(), hip.Event()
        hip.stream_sync(self.stream)
        wall0 = time.perf_counter()
        e0.record(self.stream)
        for t in range(W, W + K):
            self.step(t)
        e1.record(self.stream)
        e1.synchronize()
        wall = time.perf_counter() - wall0
        ms = e0.elapsed_ms(e1)
        assert self.be.device_status() == ffi.BackendResult.OK
        e0.close()
        e1.close()
        return ms, wall

    def ffi_rate(self, steps: int) -> float:
        """tok/s of the synchronous host-buffer entry point (slots and tokens from host
        memory, n rows of logits back into host memory), called through the C ABI with the
        step's arrays ready, as a compiled host calls it; the library validates every call."""
        out = np.empty((self.n, self.vocab), np.float32)
        slots = np.arange(self.n, dtype=np.uint32)
        toks = [np.ascontiguousarray(t, np.uint32) for t in self.tokens]
        fn = (self.be.lib.lib.redukt_backend_forward_batch_probs if self.probs
              else self.be.lib.lib.redukt_backend_forward_batch)
        sp, op = ffi._ptr(slots, ctypes.c_uint32), ffi._ptr(out, ctypes.c_float)
        tps = [ffi._ptr(t, ctypes.c_uint32) for t in toks]
        assert fn(self.n, sp, tps[0], op, self.vocab) == 0
        t0 = time.perf_counter()
        for t in range(steps):
            rc = fn(self.n, sp, tps[t % len(tps)], op, self.vocab)
            if rc != 0:
                raise ffi.BackendError(ffi.BackendResult.from_code(rc), "forward_batch")
        return self.n * steps / (time.perf_counter() - t0)

    def cdf_sym_rate(self, steps: int) -> float:
        """tok/s of compression's device path through the C ABI: each step's forward, its
        device CDFs and the coder's three values per stream (cdf[next], cdf[next + 1], the
        total; the next symbol is the following step's token) back in host memory, each
        step queued before the previous one's values are collected
        (forward_batch_cdf_sym_submit / _wait), as the lockstep driver compresses."""
        L = self.be.lib.lib
        slots = np.arange(self.n, dtype=np.uint32)
        toks = [np.ascontiguousarray(t, np.uint32) for t in self.tokens]
        out = np.empty(3 * self.n, np.uint32)
        sp, op = ffi._ptr(slots, ctypes.c_uint32), ffi._ptr(out, ctypes.c_uint32)
        tps = [ffi._ptr(t, ctypes.c_uint32) for t in toks]
        ticket = ctypes.c_uint64(0)

        def submit(t: int) -> int:
            rc = L.redukt_backend_forward_batch_cdf_sym_submit(self.n, sp, tps[t % len(tps)],
                                                               tps[(t + 1) % len(tps)], self.vocab,
                                                               ctypes.byref(ticket))
            if rc != 0:
                raise ffi.BackendError(ffi.BackendResult.from_code(rc), "forward_batch_cdf_sym_submit")
            return ticket.value

        def wait(tk: int) -> None:
            rc = L.redukt_backend_forward_batch_cdf_sym_wait(tk, op, self.n)
            if rc != 0:
                raise ffi.BackendError(ffi.BackendResult.from_code(rc), "forward_batch_cdf_sym_wait")

        wait(submit(0))   # the CDF scratch and the step's graph exist before the clock starts
        t0 = time.perf_counter()
        pending = submit(1)
        for t in range(2, steps + 1):
            nxt = submit(t)
            wait(pending)
            pending = nxt
        wait(pending)
        return self.n * steps / (time.perf_counter() - t0)

    def close(self) -> None:
        for b in (self.d_tokens, self.d_slots, self.d_out):
            b.close()


# The grid of the metric: both weight profiles at 1, 32 and 128 streams on the matrix-core
# family, the wavefront-GEMV tier (the small-batch family) where it is competitive, and the
# reference-order tier (logits bit-identical to the CPU path) with the reference's own int8
# profile (groups of 64).
# int8 per-row also runs the large-batch workload (1024 streams) on both families, where
# the projections become 1024-column skinny GEMMs: matrix cores against wavefront GEMVs.
GRID = {"f32": (1, 32, 128), "q8row-all": (1, 32, 128, 1024), "f32-gemv": (1, 32),
        "q8row-all-gemv": (1, 32, 128, 1024), "q8-ref": (1, 32)}


def grid_rates(path: str, grid, K: int, W: int) -> dict:
    """Mamba-130M at each batch size and weight profile: device tok/s, FFI tok/s and the
    whole step's bytes over its time against the HBM peak."""
    dims = rbin.MAMBA_130M
    rng = np.random.default_rng(4321)
    out = {}
    for name, sizes in grid.items():
        profile = PROFILES[name]
        be = ffi.PluginBackend(path, 0, profile)
        out[name] = {}
        for n in sizes:
            toks = synth.zipf_tokens(rng, dims.vocab, (W + K + 1, n))
            wl = Workload(be, n, dims.vocab, toks)
            ms, _ = wl.timed(W, K)
            us = ms / K * 1e3
            sb = step_bytes(dims, profile, n)
            out[name][str(n)] = {"tok_s": round(n * K / (ms / 1e3), 1), "us_per_step": round(us, 1),
                                 "step_hbm_frac": round(sb / (us / 1e6) / 1e9 / HBM_PEAK_GBS, 4),
                                 "ffi_tok_s": round(wl.ffi_rate(max(4, min(K, 32))), 1)}
            log(f"grid {name} n={n}: {out[name][str(n)]}")
            wl.close()
        be.close()
    return out


def config_rates(mamba_path: str, K: int, W: int) -> dict:
    """The other workload configurations' device rates: Mamba-130M F32 at 128 streams
    handing back the probability vector (softmax over the vocabulary), and RWKV-7 0.1B at
    64 streams of byte-level ids, F32 and int8 weight-only per row."""
    out = {}
    rng = np.random.default_rng(5678)
    runs = [("mamba130m-f32-n128-probs", mamba_path, rbin.MAMBA_130M, "f32", 128, True, True),
            ("rwkv7-0.1b-f32-n64", None, rwkv.RWKV7_0_1B, "f32", 64, False, False),
            ("rwkv7-0.1b-q8row-n64", None, rwkv.RWKV7_0_1B, "q8row", 64, False, False)]
    for name, path, dims, prof, n, probs, mamba in runs:
        if path is None:
            path = ensure_rwkv(os.path.join(tempfile.gettempdir(), "redukt_bench", "rwkv7_0_1b.rbin"))
        profile = PROFILES[prof]
        be = ffi.PluginBackend(path, 0, profile)
        toks = (synth.zipf_tokens(rng, dims.vocab, (W + K + 1, n)) if mamba
                else rng.integers(0, 256, size=(W + K + 1, n), dtype=np.uint32))
        wl = Workload(be, n, dims.vocab, toks, probs=probs)
        ms, _ = wl.timed(W, K)
        us = ms / K * 1e3
        sb = (step_bytes(dims, profile, n) + (algorithmic_bytes(dims, profile, n)["softmax"] if probs else 0)
              if mamba else rwkv_step_bytes(dims, profile, n))
        out[name] = {"tok_s": round(n * K / (ms / 1e3), 1), "us_per_step": round(us, 1),
                     "step_hbm_frac": round(sb / (us / 1e6) / 1e9 / HBM_PEAK_GBS, 4)}
        log(f"config {name}: {out[name]}")
        wl.close()
        be.close()
    out["steps"], out["warmup"] = K, W
    return out


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=1024)
    ap.add_argument("--warmup", type=int, default=32)
    ap.add_argument("--streams", type=int, default=None, help="default 128 (Mamba), 64 (RWKV-7)")
    ap.add_argument("--arch", default="mamba130m", choices=["mamba130m", "rwkv7-0.1b"],
                    help="rwkv7-0.1b: RWKV-7 0.1B, uniform byte-level tokens (not the headline metric)")
    ap.add_argument("--profile", default="q8row-all", choices=sorted(PROFILES))
    ap.add_argument("--exact-scan", action="store_true",
                    help="Mamba scan decay factors by the reference's portable exp (profile bit 3)")
    ap.add_argument("--probe-steps", type=int, default=8)
    ap.add_argument("--cpu-seconds", type=float, default=12.0)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-grid", action="store_true",
                    help="skip the 1/32/128/1024 x F32/int8 grid and the other workload configurations")
    ap.add_argument("--copy-calibration-mib", type=int, default=0,
                    help="after the probe pass, copy this many MiB device to device on the library's "
                         "stream (a copy of known size for scaling HBM byte counters)")
    ap.add_argument("--model", default=None, help="weight file (written with synthetic weights if absent)")
    ap.add_argument("--split", type=int, default=None,
                    help="most sub-batches a step is split into, each on its own HIP stream (REDUKT_GPU_SPLIT)")
    ap.add_argument("--probs", action="store_true",
                    help="hand back the probability vector (softmax over the vocabulary) instead of logits")
    args = ap.parse_args()

    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print(f"bench.py measures one GPU: the backend serves all streams of a process on one device "
              f"(--gpus {args.gpus} is not supported; shard streams over one process per GPU instead)",
              file=sys.stderr)
        return 2
    if hip.device_count() < 1:
        print("bench.py: no GPU visible", file=sys.stderr)
        return 1
    if args.split is not None:
        os.environ["REDUKT_GPU_SPLIT"] = str(args.split)

    mamba = args.arch == "mamba130m"
    n = args.streams or (128 if mamba else 64)
    K, W = args.steps, args.warmup
    profile = PROFILES[args.profile] | (ffi.PROFILE_EXACT_SCAN if args.exact_scan else 0)
    rng = np.random.default_rng(1234)
    total = W + K + args.probe_steps + 1
    if mamba:
        dims = rbin.MAMBA_130M
        path = ensure_model(args.model or os.path.join(tempfile.gettempdir(), "redukt_bench", "mamba130m.rbin"))
        tokens = synth.zipf_tokens(rng, dims.vocab, (total, n))
        exact = "-exactscan" if args.exact_scan else ""
        vocab, workload = dims.vocab, f"mamba130m-{args.profile}{exact}-n{n}-zipf1.1{'-probs' if args.probs else ''}"
    else:
        dims = rwkv.RWKV7_0_1B
        path = ensure_rwkv(args.model or os.path.join(tempfile.gettempdir(), "redukt_bench", "rwkv7_0_1b.rbin"))
        tokens = rng.integers(0, 256, size=(total, n), dtype=np.uint32)   # byte-level ids
        vocab, workload = dims.vocab, f"rwkv7-0.1b-{args.profile}-n{n}-bytes{'-probs' if args.probs else ''}"

    be = ffi.PluginBackend(path, 0, profile)
    wl = Workload(be, n, vocab, tokens, probs=args.probs)
    stream = wl.stream
    # The 4096-token boundary (reset before forward 4097) falls on timed step K // 2.
    reset_step = K // 2
    log(f"warm-up {W} steps, n={n}, profile={args.profile}")
    ms, wall = wl.timed(W, K, reset_at=reset_step)
    tok_s = n * K / (ms / 1e3)
    log(f"timed {K} steps: {ms:.2f} ms on the stream ({ms / K * 1e3:.1f} us/step), wall {wall * 1e3:.1f} ms")

    # Probe pass, after the timed region on the same stream and pool, two ways per kernel
    # class: (1) class-only steps, all of a step's launches of the class back to back
    # between one event pair (avg_us: per-launch time with the event cost spread over the
    # launches); (2) full steps with every launch of the class recording its own dispatch
    # start and stop (dispatch_avg_us; this is the roofline figure).  Probed steps run
    # unsplit, as direct launches.
    per_class = {}
    P = args.probe_steps
    t0 = W + K

    def probe(cls: int, n_events: int) -> list:
        evs = [hip.Event() for _ in range(n_events)]
        arr = (ctypes.c_void_p * len(evs))(*[e.h for e in evs])
        be.probe_kernel(cls, arr)
        for t in range(P):
            wl.step(t0 + t % (total - t0))
        used = be.probe_used()
        be.probe_kernel(0, None)
        hip.stream_sync(stream)
        assert used == len(evs), (cls, used, len(evs))
        durs = [1e3 * evs[2 * i].elapsed_ms(evs[2 * i + 1]) for i in range(len(evs) // 2)]
        for e in evs:
            e.close()
        return durs

    classes = ffi.KERNEL_CLASSES if mamba else ffi.RWKV_KERNEL_CLASSES
    for name, cls in classes.items():
        if name == "softmax" and not args.probs:
            continue
        launches = launches_per_step(dims, name, mamba, profile)
        only = probe(cls | ffi.PROBE_CLASS_ONLY, 2 * P)
        each = probe(cls, 2 * launches * P)
        per_class[name] = {"avg_us": float(np.mean(only)) / launches, "launches_per_step": launches,
                           "us_per_step": float(np.mean(only)), "dispatch_avg_us": round(float(np.mean(each)), 2)}
    alg = algorithmic_bytes(dims, profile, n) if mamba else rwkv_algorithmic_bytes(dims, profile, n)
    dom = max(per_class, key=lambda k: per_class[k]["us_per_step"])
    # roofline.achieved: the dominant kernel's algorithmic bytes over its average launch
    # duration inside full steps (events around each launch on the library's stream, the
    # duration a kernel trace reports); the class-only figure (its launches back to back)
    # is kept beside it.
    achieved = alg[dom] / (per_class[dom]["dispatch_avg_us"] / 1e6) / 1e9
    achieved_class_only = alg[dom] / (per_class[dom]["avg_us"] / 1e6) / 1e9
    for k, v in per_class.items():
        v["alg_bytes"] = alg[k]
        v["GBps"] = round(alg[k] / (v["avg_us"] / 1e6) / 1e9, 1)
        v["avg_us"] = round(v["avg_us"], 2)
        v["us_per_step"] = round(v["us_per_step"], 2)
    log("per kernel class: " + json.dumps(per_class))

    if args.copy_calibration_mib > 0:
        # copies of known size for scaling byte counters: the runtime's copy, then the
        # library's probe copy with 4- and 16-byte lanes, default and streaming policy
        # (k_copy_probe<policy, bytes per lane>, the recurrent state's shape is <2, 4>)
        nb = args.copy_calibration_mib << 20
        src, dst = hip.DeviceBuffer(nb), hip.DeviceBuffer(nb)
        hip.copy_d2d_async(dst.ptr, src.ptr, nb, stream)
        for mode in range(4):
            assert be.lib.lib.redukt_backend_copy_probe(dst.ptr, src.ptr, nb, mode) == 0
        hip.stream_sync(stream)
        log(f"copy calibration: {nb} bytes device to device, runtime copy and 4 probe copies")
        src.close()
        dst.close()

    ffi_tok_s = wl.ffi_rate(min(64, K))
    cdf_sym_tok_s = wl.cdf_sym_rate(min(64, K)) if not args.probs else None
    wl.close()
    be.close()

    grid = configs = None
    if mamba and not args.no_grid and not args.probs and not args.exact_scan and args.model is None:
        gk, gw = max(8, min(K, 64)), max(2, min(W, 8))
        grid = grid_rates(path, GRID, gk, gw)
        grid["steps"], grid["warmup"] = gk, gw
        configs = config_rates(path, gk, gw)

    cpu = None
    if not args.no_cpu_baseline:
        log("timing the CPU oracle on the host cores")
        cpu = cpu_baseline(path, profile, n, tokens, args.cpu_seconds, mamba, args.probs)

    # HBM bytes per launch of the dominant kernel from the committed counter passes
    # (FETCH_SIZE / WRITE_SIZE scaled by a copy of known size), keyed by workload.
    traffic = None
    tpath = os.path.join(ROOT, "profiles", "hbm_traffic.json")
    if os.path.exists(tpath):
        with open(tpath) as f:
            tj = json.load(f)
        entry = tj.get("workloads", {}).get(workload)
        if entry:
            traffic = entry["bytes_per_launch"].get(dom)

    sb = step_bytes(dims, profile, n) if mamba else rwkv_step_bytes(dims, profile, n)
    if args.probs:
        sb += alg["softmax"]
    result = {
        "metric": METRIC if mamba else "RWKV-7 0.1B tok/s (lockstep streams, byte-level tokens)",
        "value": round(tok_s, 1),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": K,
        "warmup": W,
        "ms_per_step": round(ms / K, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "i8xi8->i32 + f32" if profile & ffi.PROFILE_W8A8 else "f32",
        "data": "synthetic",
        "config": {"workload": workload, "layers": dims.n_layer,
                   "d_model": dims.d_model, "vocab": vocab, "streams": n, "weight_profile": args.profile,
                   "reset_every": RESET_PERIOD, "reset_at_timed_step": reset_step,
                   "output": "probabilities" if args.probs else "logits", "parallelism": "none",
                   "split_max": int(os.environ.get("REDUKT_GPU_SPLIT", "2"))},
        "roofline": {"bound": "hbm", "kernel": dom, "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": traffic,
                     "alg_bytes": alg[dom], "avg_us": per_class[dom]["dispatch_avg_us"],
                     "achieved_class_only": round(achieved_class_only, 1),
                     "frac_class_only": round(achieved_class_only / HBM_PEAK_GBS, 4)},
        "cpu_baseline": cpu,
        "step_bytes": sb,
        "step_GBps": round(sb / (ms / K / 1e3) / 1e9, 1),
        "step_hbm_frac": round(sb / (ms / K / 1e3) / 1e9 / HBM_PEAK_GBS, 4),
        "ffi_tok_s": round(ffi_tok_s, 1),
        "cdf_sym_tok_s": round(cdf_sym_tok_s, 1) if cdf_sym_tok_s is not None else None,
        "wall_ms": round(wall * 1e3, 2),
        "kernels": per_class,
        "grid": grid,
        "configs": configs,
    }
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
