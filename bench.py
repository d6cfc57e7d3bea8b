#!/usr/bin/env python3
"""Benchmark of the gfx950 quantized-linear hot path (one MI355X).

Headline (``value``): Q4_0 x Q8_0 M=1 throughput in GB/s on BASELINE cfg3, the
TinyLlama-1.1B-shaped decode step -- 22 layers x 7 linears (q, k, v, o, gate,
up, down), each activation re-quantised to Q8_0 right before its GEMV, 545 MB
of Q4_0 weights per step (beyond the 256 MB MALL, so every step streams HBM).
A step is all 154 quantise+GEMV tasks in one batched launch (the cfg3 linears
read independent activations); the dependency-staged schedule (88 launches per
step) and one-kernel-per-linear schedule (308 launches) are reported beside it.

Also reported on the same JSON line:
  * ``roofline``      -- the batched Q4_0 kernel's achieved HBM GB/s from its own
                          per-launch device time (hipExtLaunchKernel events);
  * ``w8a8``          -- cfg4 dynamic-W8A8 prefill GEMMs (M=4096) in TOPS, whole
                          operator and GEMM-only, with an int8-MFMA roofline;
  * ``configs``       -- cfg0 (rotated over >= 512 MB of weight copies), cfg1, cfg2 (lane layout,
                         and over the native ggml rows);
  * ``q8_0_q8_0``     -- the Q8_0 x Q8_0 linear (native blocks) at M = 1 and M = 4 decode
                         shapes, rotated weights, in GB/s against the HBM peak;
  * ``q4_0_long_rows``-- Q4_0 linears over native rows of 176 to 448 blocks (K = 5632 to
                         14336) at M = 1 to 4, rotated weights;
  * ``cpu_baseline``  -- the NumPy oracle of the reference CPU path on this host.

Usage: python bench.py [--steps K] [--warmup W] [--gpus 1] [--legs decode,w8a8,gemv,prefill,geglu,q8_0,q4_long,shards,cfg0,cfg1,cfg2,copy,cpu]
Weights and activations are synthetic (seeded random, the BASELINE distributions).
"""

from __future__ import annotations

import argparse
import ctypes
import json
import os
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
for _p in (ROOT, ROOT / "qpu-xla-triton_amd"):
    if str(_p) not in sys.path:
        sys.path.insert(0, str(_p))

METRIC = "Q4_0×Q8_0 GEMV GB/s (%HBM peak); W8A8 GEMM int8 TOPS (%MFMA peak)"
PEAK_HBM_GBS = 8000.0  # MI355X HBM3E
PEAK_INT8_TOPS = 5000.0  # MI355X dense int8 MFMA, 5.0 POP/s
TINYLLAMA_LAYER = (  # (name, K, N)
    ("q", 2048, 2048),
    ("k", 2048, 256),
    ("v", 2048, 256),
    ("o", 2048, 2048),
    ("gate", 2048, 5632),
    ("up", 2048, 5632),
    ("down", 5632, 2048),
)
LAYERS = 22
ROTATION_BYTES = 512 << 20


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def q4_linear_bytes(m: int, k: int, n: int) -> int:
    """Algorithmic bytes of one Q4_0 x Q8_0 linear: weights + Q8_0 activation + fp32 output."""
    return n * (k // 32) * 18 + m * (k // 32) * 34 + m * n * 4


def parse_args() -> argparse.Namespace:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--legs", default="decode,w8a8,gemv,prefill,geglu,q8_0,q4_long,shards,cfg0,cfg1,cfg2,copy,cpu")
    ap.add_argument("--cpu-seconds", type=float, default=10.0, help="budget of each CPU-baseline sample")
    return ap.parse_args()


class Runner:
    """Prebuilt ctypes calls on one stream, replayable eagerly or as a captured HIP graph.

    The operands are made on torch's current stream, the launches go to
    ``stream``: the first launch waits for the whole device (every producer
    queued so far), and ``uses`` marks tensors as used on ``stream`` so the
    caching allocator does not hand their blocks out again while launches on
    it are pending.
    """

    def __init__(self, torch, stream) -> None:
        from qpu_xla_amd import _lib

        self.torch = torch
        self.stream = stream
        self.lib = _lib.load()
        self._lib = _lib
        self.calls: list[tuple[object, tuple]] = []
        self.handle = ctypes.c_void_p(int(stream.cuda_stream))
        self._ordered = False

    def add(self, name: str, *args) -> None:
        self.calls.append((getattr(self.lib, name), args))

    def uses(self, *tensors) -> None:
        for t in tensors:
            t.record_stream(self.stream)

    def _order_after_producers(self) -> None:
        if not self._ordered:
            self.torch.cuda.synchronize()
            self._ordered = True

    def run(self) -> None:
        self._order_after_producers()
        for fn, args in self.calls:
            rc = fn(*args)
            if rc:
                self._lib.check(rc)

    def capture(self):
        torch = self.torch
        graph = torch.cuda.CUDAGraph()
        self._order_after_producers()
        torch.cuda.synchronize()
        with torch.cuda.graph(graph, stream=self.stream):
            self.run()
        torch.cuda.synchronize()
        return graph

    def timed_graph(self, graph, steps: int, warmup: int) -> tuple[float, float]:
        """(wall ms per replay, event ms per replay), synchronised on both sides."""
        torch = self.torch
        with torch.cuda.stream(self.stream):
            for _ in range(warmup):
                graph.replay()
            torch.cuda.synchronize()
            start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            t0 = time.perf_counter()
            start.record(self.stream)
            for _ in range(steps):
                graph.replay()
            end.record(self.stream)
            torch.cuda.synchronize()
            wall = (time.perf_counter() - t0) * 1e3 / steps
        return wall, start.elapsed_time(end) / steps

    def capture_steps(self, steps: int):
        """One graph holding `steps` consecutive steps (each step's launches in order)."""
        torch = self.torch
        graph = torch.cuda.CUDAGraph()
        self._order_after_producers()
        torch.cuda.synchronize()
        with torch.cuda.graph(graph, stream=self.stream):
            for _ in range(steps):
                self.run()
        torch.cuda.synchronize()
        return graph

    def timed_once(self, graph, warmup: int) -> tuple[float, float]:
        """(wall ms, event ms) of one replay of `graph`, after `warmup` replays."""
        torch = self.torch
        with torch.cuda.stream(self.stream):
            for _ in range(warmup):
                graph.replay()
            torch.cuda.synchronize()
            start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            t0 = time.perf_counter()
            start.record(self.stream)
            graph.replay()
            end.record(self.stream)
            torch.cuda.synchronize()
            wall = (time.perf_counter() - t0) * 1e3
        return wall, start.elapsed_time(end)

    def timed_eager(self, steps: int, warmup: int) -> tuple[float, float]:
        """(wall ms per step, event ms per step) of eager back-to-back launches."""
        torch = self.torch
        for _ in range(warmup):
            self.run()
        torch.cuda.synchronize()
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        t0 = time.perf_counter()
        start.record(self.stream)
        for _ in range(steps):
            self.run()
        end.record(self.stream)
        torch.cuda.synchronize()
        wall = (time.perf_counter() - t0) * 1e3 / steps
        return wall, start.elapsed_time(end) / steps

    def kernel_times(self, repeats: int = 1) -> dict[str, list[float]]:
        """Device time of every launch of ``repeats`` eager runs, grouped by kernel name."""
        out: dict[str, list[float]] = {}
        with self._lib.launch_timing() as timing:
            for _ in range(repeats):
                self.run()
        for name, ms in timing.records:
            out.setdefault(name, []).append(ms)
        return out


def _p(t) -> ctypes.c_void_p:
    return ctypes.c_void_p(t.data_ptr())


def _rs(t) -> int:
    return int(t.stride(0)) * t.element_size()


# ------------------------------------------------------------ output checks
# After its timed region, every leg checks outputs of the launches it timed
# against a torch restatement of the reference arithmetic on the host: exact
# integer dots and the same fp32 roundings in the same order, so the check is
# bit-exact.  (The NumPy oracle is test infrastructure; only the CPU-baseline
# legs run it.)  A mismatch stops the run.


def _fp16_field(torch, blocks):
    return blocks[..., 0:2].contiguous().view(torch.float16)[..., 0].float()


def _mismatch(torch, label: str, r: int, got, want, inputs: dict, others: dict | None = None) -> RuntimeError:
    """The error for a failed check: which columns differ, their bits, and non-finite inputs.

    NaN never equals NaN, so a NaN in an input (a bias, a scale) fails the
    check even where the kernel computed the same NaN; the message says so.
    ``others`` maps labels to outputs the differing columns are compared
    with (another weight copy's result, say).
    """
    diff = (got != want).nonzero().flatten()
    cols = diff[:8].tolist()
    bits = lambda t, c: f"{int(t[c:c + 1].view(torch.int32)[0]) & 0xFFFFFFFF:08x}"  # noqa: E731
    detail = ", ".join(f"col {c}: got {bits(got, c)} want {bits(want, c)}" for c in cols)
    both_nan = int((torch.isnan(got) & torch.isnan(want)).sum())
    nonfinite = {name: int((~torch.isfinite(t)).sum()) for name, t in inputs.items() if t is not None}
    msg = (f"{label}: row {r}: {diff.numel()} of {want.numel()} outputs differ from the reference arithmetic "
           f"({detail}; NaN in both at {both_nan} of them; non-finite inputs {nonfinite})")
    for name, other in (others or {}).items():
        same = int((other[diff] == got[diff]).sum())
        msg += f"; {same} of the differing columns equal {name}"
    log(msg)
    return RuntimeError(msg)


def check_q4_0(torch, label: str, q8_blocks, q4_blocks, output, rows=(0,)) -> dict:
    """output[r, :N] == sum_b fl32(fl32(float(dot_b) * dw) * da) in block order, for r in rows."""
    w = q4_blocks.cpu()
    dw = _fp16_field(torch, w)  # [N, B]
    codes = w[..., 2:].to(torch.int32)
    qw = torch.cat([(codes & 15) - 8, (codes >> 4) - 8], dim=-1)  # [N, B, 32]
    for r in rows:
        a = q8_blocks[r].cpu()
        da = _fp16_field(torch, a)  # [B]
        qa = a[..., 2:].view(torch.int8).to(torch.int32)  # [B, 32]
        dots = (qw * qa).sum(-1)  # [N, B], exact
        acc = torch.zeros(w.shape[0], dtype=torch.float32)
        for b in range(w.shape[1]):
            acc = acc + (dots[:, b].float() * dw[:, b]) * da[b]
        got = output[r, : w.shape[0]].cpu()
        if not torch.equal(got, acc):
            raise _mismatch(torch, label, r, got, acc, {"weight scales": dw, "activation scales": da})
    return {"rows_checked": list(rows), "columns": int(w.shape[0]), "bit_exact": True}


def check_w8a8(torch, label: str, x, qa, sa, weight, bias, y, rows=(0,), others: dict | None = None) -> dict:
    """Row quantiser (scale floor 1/127, rint of the true quotient) and acc*sa*sw + bias, bit for bit.

    ``others`` maps labels to other outputs [M, N] (another weight copy's
    result, say) that a mismatch report compares the differing columns with.
    """
    values = weight.values.cpu().to(torch.int64)
    sw = weight.scales.cpu()
    b = None if bias is None else bias.cpu()
    floor = torch.tensor(1.0 / 127.0, dtype=torch.float32)
    for r in rows:
        xr = x[r].cpu()
        scale = torch.maximum(xr.abs().max() / 127.0, floor)
        q = torch.clamp(torch.round(xr / scale), -127, 127).to(torch.int8)
        if not torch.equal(qa[r, : xr.numel()].cpu(), q) or not torch.equal(sa[r].cpu(), scale):
            raise RuntimeError(f"{label}: row {r}: quantised activation differs from the reference rule")
        acc = (values @ q.to(torch.int64)).to(torch.float32)
        want = (acc * scale) * sw
        if b is not None:
            want = want + b
        got = y[r].cpu()
        if not torch.equal(got, want):
            raise _mismatch(torch, label, r, got, want, {"x": xr, "column scales": sw, "bias": b},
                            {name: o[r].cpu() for name, o in (others or {}).items()})
    return {"rows_checked": list(rows), "columns": int(sw.numel()), "bit_exact": True}


def q8_0_host(torch, values):
    """fp32 rows [R, K] -> Q8_0 blocks [R, K/32, 34] on the host: d = absmax/127, q = clamp(rint(x * (1/d)))."""
    v = values.cpu().reshape(values.shape[0], -1, 32)
    d = v.abs().amax(dim=2) / 127.0
    inv = torch.where(d != 0, 1.0 / d, torch.zeros_like(d))
    q = torch.clamp(torch.round(v * inv[..., None]), -127, 127).to(torch.int8)
    out = torch.empty((v.shape[0], v.shape[1], 34), dtype=torch.uint8)
    out[..., 0:2] = d.half().view(torch.uint8).reshape(v.shape[0], v.shape[1], 2)
    out[..., 2:] = q.view(torch.uint8)
    return out


# --------------------------------------------------------------------- legs


def _decode_model(torch, gen):
    """cfg3 tensors: per linear (k, n, Q4_0 weight, its lane-layout copy, fp32 activation, Q8_0 buffer, output).

    The lane layout is the decode kernels' prepared weight form (same bytes,
    re-laid out once at load time, outside every timed region).
    """
    from qpu_xla_amd.kernels.ggml_q4_0 import pack_ggml_q4_0_lane_weights
    from qpu_xla_amd.kernels.quantize import quantize_q4_0

    model = []
    for _layer in range(LAYERS):
        layer = []
        for name, k, n in TINYLLAMA_LAYER:
            w = torch.randn((n, k), generator=gen, device="cuda", dtype=torch.float32) * 0.02
            wq = quantize_q4_0(w)
            del w
            x = torch.randn((1, k), generator=gen, device="cuda", dtype=torch.float32)
            xq = torch.empty((1, k // 32, 34), dtype=torch.uint8, device="cuda")
            y = torch.empty((1, n), dtype=torch.float32, device="cuda")
            layer.append({"name": name, "k": k, "n": n, "weight": wq, "lanes": pack_ggml_q4_0_lane_weights(wq),
                          "x": x, "xq": xq, "y": y})
        model.append(layer)
    torch.cuda.synchronize()
    return model


# Dependency stages of one transformer layer: projections in a stage read the same
# (or an independent) input; a stage needs the previous stage's output.
LAYER_STAGES = (("q", "k", "v"), ("o",), ("gate", "up"), ("down",))


def leg_decode(torch, args) -> dict:
    """cfg3: 22 x 7 Q4_0 linears at M=1, each activation quantised to Q8_0 before its GEMV.

    Three schedules of the same 154 quantise+GEMV tasks:
      batched    -- one batch per step: a Q8_0 pre-pass launch quantising all 154
                    fp32 activations, then one grid over every linear's column
                    tiles; the cfg3 linears read independent activations, so the
                    whole step is one batch;
      staged     -- one launch per dependency stage (q/k/v, o, gate/up, down):
                    88 launches per step, the order a real decode step needs;
      per_linear -- a Q8_0 quantise kernel + a GEMV kernel per linear: 308 launches.
    Each schedule is replayed as one HIP graph per step.
    """
    from qpu_xla_amd.kernels.ggml_q4_0 import Q4_0LinearBatch

    gen = torch.Generator(device="cuda")
    gen.manual_seed(3)
    model = _decode_model(torch, gen)
    linears = [lin for layer in model for lin in layer]
    bytes_step = sum(q4_linear_bytes(1, lin["k"], lin["n"]) for lin in linears)
    # The batch kernel reads the Q4_0 weights and the pre-pass's Q8_0 blocks and
    # writes the fp32 outputs: exactly the per-step bytes.  The pre-pass reads
    # the fp32 activations and writes the Q8_0 blocks.
    kernel_bytes = bytes_step
    prepass_bytes = sum(lin["k"] * 4 + lin["k"] // 32 * 34 for lin in linears)
    log(f"decode: {len(linears)} linears, {bytes_step / 1e6:.1f} MB per step")
    result = {"bytes_per_step": bytes_step}

    def task(lin, layout="lanes"):
        return {"x": lin["x"], "weight": lin[layout if layout == "lanes" else "weight"], "destination": lin["y"]}

    stream = torch.cuda.Stream()
    # The same batch over the native ggml weight rows, for comparison.
    native = Q4_0LinearBatch([task(lin, "native") for lin in linears])
    runner = Runner(torch, stream)
    runner.add("qxt_q4_0_batch_launch", native._handle, runner.handle)
    runner.run()
    torch.cuda.synchronize()
    ntimes = runner.kernel_times(repeats=max(3, args.steps // 2))["q4_0_batch_kernel"]
    native.close()
    result["batched_native_layout"] = {
        "kernel_avg_us": float(np.mean(ntimes)) * 1e3,
        "kernel_gbs": kernel_bytes / (float(np.mean(ntimes)) * 1e-3) / 1e9,
    }
    log(f"decode batched, native weight layout: {result['batched_native_layout']}")

    # batched: one launch per step (lane-layout weights).
    batch = Q4_0LinearBatch([task(lin) for lin in linears])
    runner = Runner(torch, stream)
    runner.add("qxt_q4_0_batch_launch", batch._handle, runner.handle)
    runner.run()
    torch.cuda.synchronize()
    all_times = runner.kernel_times(repeats=max(3, args.steps // 2))
    times = all_times["q4_0_batch_kernel"]
    prepass = all_times.get("q8_0_prepass_kernel", [0.0])
    graph = runner.capture()
    graph_wall, graph_events = runner.timed_graph(graph, args.steps, args.warmup)
    del graph
    eager_wall, eager_events = runner.timed_eager(args.steps, args.warmup)
    # All K steps captured back to back in one graph: the same K launches,
    # without a graph launch (or a Python call) between consecutive steps.
    multi = runner.capture_steps(args.steps)
    multi_wall, multi_events = runner.timed_once(multi, max(1, args.warmup // args.steps))
    del multi
    modes = {
        "graph_per_step": (graph_wall, graph_events),
        "eager": (eager_wall, eager_events),
        "graph_of_k_steps": (multi_wall / args.steps, multi_events / args.steps),
    }
    # Every mode runs exactly K full steps; the line reports the fastest way of issuing them.
    mode = min(modes, key=lambda name: modes[name][0])
    wall_ms, event_ms = modes[mode]
    kernel_ms = float(np.mean(times))
    result["batched"] = {
        "weight_layout": "lanes",
        "launches_per_step": 2,
        "work_items": batch.work_items,
        "launch_mode": mode,
        "ms_per_step_wall": wall_ms,
        "ms_per_step_events": event_ms,
        "ms_per_step_wall_by_mode": {name: value[0] for name, value in modes.items()},
        "gbs": bytes_step / (wall_ms * 1e-3) / 1e9,
        "kernel_avg_us": kernel_ms * 1e3,
        "kernel_min_us": float(np.min(times)) * 1e3,
        "kernel_bytes_per_launch": kernel_bytes,
        "kernel_gbs": kernel_bytes / (kernel_ms * 1e-3) / 1e9,
        "prepass_avg_us": float(np.mean(prepass)) * 1e3,
        "prepass_bytes_per_launch": prepass_bytes,
    }
    torch.cuda.synchronize()
    result["batched"]["check"] = {
        f"linear_{i}": check_q4_0(torch, f"decode batched linear {i}", q8_0_host(torch, linears[i]["x"]),
                                  linears[i]["weight"], linears[i]["y"])
        for i in (0, len(linears) // 2, len(linears) - 1)
    }
    log(f"decode batched: {result['batched']}")

    # staged: one batch per dependency stage.
    stages = []
    for layer in model:
        by_name = {lin["name"]: lin for lin in layer}
        for names in LAYER_STAGES:
            stages.append(Q4_0LinearBatch([task(by_name[nm]) for nm in names]))
    runner = Runner(torch, stream)
    for st in stages:
        runner.add("qxt_q4_0_batch_launch", st._handle, runner.handle)
    runner.run()
    torch.cuda.synchronize()
    stimes = runner.kernel_times(repeats=2)["q4_0_batch_kernel"]
    graph = runner.capture()
    wall_ms, event_ms = runner.timed_graph(graph, args.steps, args.warmup)
    result["staged"] = {
        "launches_per_step": len(stages),
        "ms_per_step_wall": wall_ms,
        "ms_per_step_events": event_ms,
        "gbs": bytes_step / (wall_ms * 1e-3) / 1e9,
        "kernel_sum_us_per_step": float(np.sum(stimes)) * 1e3 / 2,
    }
    del graph
    torch.cuda.synchronize()
    last = linears[-1]
    result["staged"]["check"] = check_q4_0(torch, "decode staged", q8_0_host(torch, last["x"]), last["weight"], last["y"])
    log(f"decode staged: {result['staged']}")

    # per_linear: quantise kernel + GEMV kernel per linear.
    runner = Runner(torch, stream)
    for lin in linears:
        x, xq, lw, y, k, n = lin["x"], lin["xq"], lin["lanes"], lin["y"], lin["k"], lin["n"]
        runner.add("qxt_quantize_q8_0", _p(x), _rs(x), _p(xq), _rs(xq), 1, k, runner.handle)
        runner.add("qxt_ggml_q4_0_q8_0_linear_lanes", _p(xq), _rs(xq), _p(lw.packed), n, _p(y), _rs(y),
                   1, k // 32, 0, 0, n, runner.handle)
    runner.run()
    torch.cuda.synchronize()
    ptimes = runner.kernel_times(repeats=2)
    graph = runner.capture()
    wall_ms, event_ms = runner.timed_graph(graph, args.steps, args.warmup)
    q4_times = ptimes.get("q4_0_linear_kernel", [])
    result["per_linear"] = {
        "launches_per_step": len(runner.calls),
        "ms_per_step_wall": wall_ms,
        "ms_per_step_events": event_ms,
        "gbs": bytes_step / (wall_ms * 1e-3) / 1e9,
        "q4_linear_avg_us": float(np.mean(q4_times)) * 1e3,
        "q4_linear_kernel_gbs": bytes_step / len(linears) / (float(np.mean(q4_times)) * 1e-3) / 1e9,
        "q8_0_avg_us": float(np.mean(ptimes.get("q8_0_kernel", [0.0]))) * 1e3,
    }
    del graph
    torch.cuda.synchronize()
    result["per_linear"]["check"] = check_q4_0(torch, "decode per_linear", q8_0_host(torch, last["x"]),
                                               last["weight"], last["y"])
    log(f"decode per_linear: {result['per_linear']}")
    batch.close()
    for st in stages:
        st.close()
    del model, linears
    torch.cuda.synchronize()
    torch.cuda.empty_cache()
    return result


def leg_rotated_q4(torch, args, rows: int, k: int, n: int, seed: int, layout: str = "lanes") -> dict:
    """One Q4_0 linear shape, cycling through >= 512 MB of distinct weight copies.

    layout "lanes": the decode kernels' prepared lane layout; "native": the ggml rows as given.
    """
    from qpu_xla_amd.kernels.ggml_q4_0 import pack_ggml_q4_0_lane_weights
    from qpu_xla_amd.kernels.quantize import quantize_q4_0, quantize_q8_0

    gen = torch.Generator(device="cuda")
    gen.manual_seed(seed)
    per = n * (k // 32) * 18
    copies = max(2, -(-ROTATION_BYTES // per))
    stream = torch.cuda.Stream()
    runner = Runner(torch, stream)
    weights = []
    for _ in range(copies):
        w = torch.randn((n, k), generator=gen, device="cuda", dtype=torch.float32) * 0.02
        last_native = quantize_q4_0(w)  # kept for the output check of the last launch
        weights.append(pack_ggml_q4_0_lane_weights(last_native) if layout == "lanes" else last_native)
        del w
    x = torch.randn((rows, k), generator=gen, device="cuda", dtype=torch.float32)
    xq = quantize_q8_0(x)
    y = torch.empty((rows, n), dtype=torch.float32, device="cuda")
    for lw in weights:
        if layout == "lanes":
            runner.add("qxt_ggml_q4_0_q8_0_linear_lanes", _p(xq), _rs(xq), _p(lw.packed), n, _p(y), _rs(y),
                       rows, k // 32, 0, 0, n, runner.handle)
        else:
            runner.add("qxt_ggml_q4_0_q8_0_linear", _p(xq), _rs(xq), _p(lw), _rs(lw), _p(y), _rs(y),
                       rows, k // 32, 0, 0, n, runner.handle)
    runner.run()
    torch.cuda.synchronize()
    times = runner.kernel_times(repeats=2)["q4_0_linear_kernel"]
    graph = runner.capture()
    wall_ms, _ = runner.timed_graph(graph, max(2, args.steps // 4), 2)
    b = q4_linear_bytes(rows, k, n)
    avg_ms = float(np.mean(times))
    out = {
        "shape": f"M={rows} K={k} N={n}",
        "weight_layout": layout,
        "copies": copies,
        "rotation_mb": copies * per / 1e6,
        "bytes_per_launch": b,
        "kernel_avg_us": avg_ms * 1e3,
        "kernel_gbs": b / (avg_ms * 1e-3) / 1e9,
        "kernel_frac_hbm": b / (avg_ms * 1e-3) / 1e9 / PEAK_HBM_GBS,
        "stream_us_per_launch": wall_ms * 1e3 / copies,
        "stream_gbs": b * copies / (wall_ms * 1e-3) / 1e9,
    }
    torch.cuda.synchronize()
    out["check"] = check_q4_0(torch, out["shape"], q8_0_host(torch, x), last_native, y, rows=tuple(range(rows)))
    del graph, weights, last_native
    torch.cuda.synchronize()
    torch.cuda.empty_cache()
    return out


def q8_linear_bytes(m: int, k: int, n: int) -> int:
    """Algorithmic bytes of one Q8_0 x Q8_0 linear: weights + Q8_0 activation + fp32 output."""
    return n * (k // 32) * 34 + m * (k // 32) * 34 + m * n * 4


def check_q8_0_q8_0(torch, label: str, act_blocks, w_blocks, output, rows=(0,)) -> dict:
    """output[r, :N] == sum_b fl32(fl32(float(dot_b) * da) * dw) in block order (activation scale first)."""
    w = w_blocks.cpu()
    dw = _fp16_field(torch, w)  # [N, B]
    qw = w[..., 2:].view(torch.int8).to(torch.int32)  # [N, B, 32]
    for r in rows:
        a = act_blocks[r].cpu()
        da = _fp16_field(torch, a)  # [B]
        qa = a[..., 2:].view(torch.int8).to(torch.int32)  # [B, 32]
        dots = (qw * qa).sum(-1)  # [N, B], exact
        acc = torch.zeros(w.shape[0], dtype=torch.float32)
        for b in range(w.shape[1]):
            acc = acc + (dots[:, b].float() * da[b]) * dw[:, b]
        got = output[r, : w.shape[0]].cpu()
        if not torch.equal(got, acc):
            raise _mismatch(torch, label, r, got, acc, {"weight scales": dw, "activation scales": da})
    return {"rows_checked": list(rows), "columns": int(w.shape[0]), "bit_exact": True}


def leg_rotated_q8(torch, args, rows: int, k: int, n: int, seed: int) -> dict:
    """One Q8_0 x Q8_0 linear shape (native 34-byte blocks on both sides), cycling through
    >= 512 MB of distinct weight copies so that every launch streams its weights from HBM."""
    from qpu_xla_amd.kernels.quantize import quantize_q8_0

    gen = torch.Generator(device="cuda")
    gen.manual_seed(seed)
    per = n * (k // 32) * 34
    copies = max(2, -(-ROTATION_BYTES // per))
    runner = Runner(torch, torch.cuda.Stream())
    weights = []
    for _ in range(copies):
        w = torch.randn((n, k), generator=gen, device="cuda", dtype=torch.float32) * 0.02
        weights.append(quantize_q8_0(w))
        del w
    x = torch.randn((rows, k), generator=gen, device="cuda", dtype=torch.float32)
    xq = quantize_q8_0(x)
    y = torch.empty((rows, n), dtype=torch.float32, device="cuda")
    runner.uses(xq, y, *weights)
    for wq in weights:
        runner.add("qxt_ggml_q8_0_q8_0_linear", _p(xq), _rs(xq), _p(wq), _rs(wq), _p(y), _rs(y),
                   rows, k // 32, 0, 0, n, runner.handle)
    runner.run()
    torch.cuda.synchronize()
    times = runner.kernel_times(repeats=2)["q8_0_linear_kernel"]
    graph = runner.capture()
    wall_ms, _ = runner.timed_graph(graph, max(2, args.steps // 4), 2)
    b = q8_linear_bytes(rows, k, n)
    avg_ms = float(np.mean(times))
    out = {
        "shape": f"M={rows} K={k} N={n}",
        "copies": copies,
        "rotation_mb": copies * per / 1e6,
        "bytes_per_launch": b,
        "kernel_avg_us": avg_ms * 1e3,
        "kernel_gbs": b / (avg_ms * 1e-3) / 1e9,
        "kernel_frac_hbm": b / (avg_ms * 1e-3) / 1e9 / PEAK_HBM_GBS,
        "stream_us_per_launch": wall_ms * 1e3 / copies,
        "stream_gbs": b * copies / (wall_ms * 1e-3) / 1e9,
    }
    torch.cuda.synchronize()
    out["check"] = check_q8_0_q8_0(torch, "q8_0 " + out["shape"], xq, weights[-1], y, rows=tuple(range(rows)))
    del graph, weights
    torch.cuda.synchronize()
    torch.cuda.empty_cache()
    return out


def gemm_kernel_ms(times: dict[str, list[float]]) -> float:
    """Total device ms of the W8A8 GEMM launches (256 x 256 stream kernel and the tiled kernel)."""
    return float(sum(np.sum(v) for name, v in times.items() if name.startswith("w8a8_gemm")))


def _w8a8_operands(torch, gen, m: int, k: int, n: int):
    from qpu_xla_amd.quantization import quantize_per_output_channel_int8

    x = torch.randn((m, k), generator=gen, device="cuda", dtype=torch.float32)
    outliers = torch.randperm(k, generator=gen, device="cuda")[: max(1, round(0.001 * k))]
    x[:, outliers] *= 20.0
    w = torch.randn((n, k), generator=gen, device="cuda", dtype=torch.float32) * 0.02
    weight = quantize_per_output_channel_int8(w)
    del w
    bias = torch.randn((n,), generator=gen, device="cuda", dtype=torch.float32) * 0.1
    return x, weight, bias


def leg_w8a8(torch, args, shapes: dict | None = None) -> dict:
    """cfg4: dynamic W8A8 prefill GEMMs at Llama-3-8B FFN shapes, M=4096 (or the given shapes)."""
    gen = torch.Generator(device="cuda")
    gen.manual_seed(4)
    if shapes is None:
        shapes = {"gate_up": (4096, 4096, 14336), "down": (4096, 14336, 4096)}
    result = {}
    total_ops = 0
    total_ms = 0.0
    total_gemm_ms = 0.0
    for label, (m, k, n) in shapes.items():
        x, weight, bias = _w8a8_operands(torch, gen, m, k, n)
        qa = torch.empty((m, k), dtype=torch.int8, device="cuda")
        sa = torch.empty((m,), dtype=torch.float32, device="cuda")
        y = torch.empty((m, n), dtype=torch.float32, device="cuda")
        stream = torch.cuda.Stream()
        runner = Runner(torch, stream)
        runner.uses(x, qa, sa, weight.values, weight.scales, bias, y)
        runner.add("qxt_w8a8_linear", _p(x), _rs(x), _p(qa), _rs(qa), _p(sa), _p(weight.values),
                   _rs(weight.values), _p(weight.scales), _p(bias), _p(y), _rs(y), m, n, k, 0, 0, runner.handle)
        runner.run()
        torch.cuda.synchronize()
        # Ten or more operator calls back to back, each launch timed on the device:
        # the GEMM at the clock the board holds under sustained prefill load.
        reps = max(10, args.steps // 2)
        times = runner.kernel_times(repeats=reps)
        graph = runner.capture()
        # The operator (row quantiser + GEMM) issued back to back, as graph replays
        # and as eager launches; the faster way of issuing it is reported.
        modes = {"graph": runner.timed_graph(graph, reps, 2)[0], "eager": runner.timed_eager(reps, 2)[0]}
        mode = min(modes, key=modes.get)
        wall_ms = modes[mode]
        ops = 2 * m * n * k
        # Per operator call (a GEMM may be two launches: full tiles + a half-tile round).
        gemm_ms = gemm_kernel_ms(times) / reps
        quant_ms = float(np.sum(times["rows_int8_kernel"])) / reps
        result[label] = {
            "shape": f"M={m} K={k} N={n}",
            "operator_ms": wall_ms,
            "operator_tops": ops / (wall_ms * 1e-3) / 1e12,
            "operator_ms_by_mode": modes,
            "launch_mode": mode,
            "gemm_ms": gemm_ms,
            "gemm_tops": ops / (gemm_ms * 1e-3) / 1e12,
            "gemm_frac_mfma": ops / (gemm_ms * 1e-3) / 1e12 / PEAK_INT8_TOPS,
            "row_quantise_ms": quant_ms,
        }
        torch.cuda.synchronize()
        result[label]["check"] = check_w8a8(torch, f"w8a8 {label}", x, qa, sa, weight, bias, y, rows=(0, m - 1))
        total_ops += ops
        total_ms += wall_ms
        total_gemm_ms += gemm_ms
        del graph, x, weight, bias, qa, sa, y
        torch.cuda.synchronize()
        torch.cuda.empty_cache()
    gemm_tops = total_ops / (total_gemm_ms * 1e-3) / 1e12
    result["value"] = total_ops / (total_ms * 1e-3) / 1e12
    result["unit"] = "TOPS"
    result["roofline"] = {
        "bound": "mfma",
        "kernel": "w8a8_gemm_stream_kernel",
        "achieved": gemm_tops,
        "peak": PEAK_INT8_TOPS,
        "unit": "TOPS",
        "frac": gemm_tops / PEAK_INT8_TOPS,
        "ops_per_launch": total_ops // 2,
    }
    return result


def leg_shards(torch, args) -> dict:
    """One GPU's share of the 8-GPU shardings the path would use (the collectives are not run).

    Q4_0 shards by output columns (the reference's wcol0 / ocol0 / ncols
    partition): cfg0's N = 5632 over 8 GPUs is N = 704 per GPU, rotated
    weights.  W8A8 shards by rows with replicated weights: cfg4's M = 4096 over
    8 GPUs is M = 512 per GPU at the full K and N.
    """
    return {
        "q4_0_cfg0_column_shard": leg_rotated_q4(torch, args, 1, 2048, 704, 10),
        "w8a8_cfg4_row_shard": leg_w8a8(torch, args, {"gate_up": (512, 4096, 14336), "down": (512, 14336, 4096)}),
    }


def leg_w8a8_gemv(torch, args) -> dict:
    """Dynamic W8A8 at M = 1 (a decode token through the cfg4 FFN weights): the dot4 GEMV path.

    HBM-bound on the int8 weights; the launches cycle through >= 512 MB of
    distinct weight copies so every launch streams HBM.
    """
    gen = torch.Generator(device="cuda")
    gen.manual_seed(5)
    out = {}
    for label, (k, n) in {"gate_up": (4096, 14336), "down": (14336, 4096)}.items():
        per = n * k
        copies = max(2, -(-ROTATION_BYTES // per))
        weights = []
        from qpu_xla_amd.quantization import quantize_per_output_channel_int8

        for _ in range(copies):
            weights.append(quantize_per_output_channel_int8(torch.randn((n, k), generator=gen, device="cuda") * 0.02))
        x = torch.randn((1, k), generator=gen, device="cuda")
        bias = torch.randn((n,), generator=gen, device="cuda") * 0.1
        qa = torch.empty((1, k), dtype=torch.int8, device="cuda")
        sa = torch.empty((1,), dtype=torch.float32, device="cuda")
        # One output per weight copy, so each checked copy's result stands alone.
        ys = [torch.empty((1, n), dtype=torch.float32, device="cuda") for _ in weights]
        runner = Runner(torch, torch.cuda.Stream())
        runner.uses(x, bias, qa, sa, *ys)
        for wt, y in zip(weights, ys):
            runner.uses(wt.values, wt.scales)
            runner.add("qxt_w8a8_linear", _p(x), _rs(x), _p(qa), _rs(qa), _p(sa), _p(wt.values), _rs(wt.values),
                       _p(wt.scales), _p(bias), _p(y), _rs(y), 1, n, k, 0, 0, runner.handle)
        runner.run()
        torch.cuda.synchronize()
        # Five passes over the copies (50 event-timed launches): a single
        # launch's device time varies by several percent from launch to launch.
        times = runner.kernel_times(repeats=5)
        gemv_us = float(np.mean(times["w8a8_gemv_kernel"])) * 1e3
        graph = runner.capture()
        wall_ms, _ = runner.timed_graph(graph, max(2, args.steps // 4), 2)
        b = n * k + k + 4 * n * 3  # int8 weights + int8 activation + sw, bias, y
        out[label] = {
            "shape": f"M=1 K={k} N={n}",
            "copies": copies,
            "gemv_kernel_us": gemv_us,
            "gemv_kernel_gbs": b / (gemv_us * 1e-6) / 1e9,
            "gemv_frac_hbm": b / (gemv_us * 1e-6) / 1e9 / PEAK_HBM_GBS,
            "operator_us": wall_ms * 1e3 / copies,
            # M <= 4 quantises inside the GEMV kernel: one launch per operator call.
            "launches_per_call": sum(len(v) for v in times.values()) // (5 * copies),
        }
        torch.cuda.synchronize()
        checked = sorted({0, copies // 2, copies - 1})
        out[label]["check"] = {
            f"copy_{j}": check_w8a8(torch, f"w8a8 gemv {label} copy {j}", x, qa, sa, weights[j], bias, ys[j],
                                    others={f"copy {i}": ys[i] for i in checked if i != j})
            for j in checked
        }
        del graph, weights, ys
        torch.cuda.synchronize()
        torch.cuda.empty_cache()
    return out


def leg_prefill(torch, args) -> dict:
    """Q4_0 x Q8_0 prefill (M = 512 tokens) at the TinyLlama FFN shapes: the matrix-core path.

    Every output needs, per 32-element block, an exact int32 dot (one MFMA per
    32 x 32 outputs) and four fp32 VALU operations (convert, x dw, x da, add in
    block order), so the kernel's floor is the non-packed fp32 VALU rate:
    256 CU x 4 SIMD x 16 lanes x 2.4 GHz = 39.3 T operations/s.  Two operand
    layouts: the native 18/34-byte blocks (qxt_ggml_q4_0_q8_0_linear) and the
    split planes of the reference's tiled kernel contract, the weight packed
    once outside the timed region as the reference prepares it
    (qxt_ggml_q4_0_q8_0_tiled_linear).
    """
    from qpu_xla_amd.kernels.ggml_q4_0 import pack_ggml_q4_0_tiled_weights, split_ggml_q8_0_blocks
    from qpu_xla_amd.kernels.quantize import quantize_q4_0, quantize_q8_0

    gen = torch.Generator(device="cuda")
    gen.manual_seed(6)
    rows = 512
    valu_peak = 256 * 4 * 16 * 2.4e9
    out = {}
    for label, (k, n) in {"gate_up": (2048, 5632), "down": (5632, 2048)}.items():
        wq = quantize_q4_0(torch.randn((n, k), generator=gen, device="cuda") * 0.02)
        x = torch.randn((rows, k), generator=gen, device="cuda")
        xq = quantize_q8_0(x)
        w_scales, w_words = pack_ggml_q4_0_tiled_weights(wq)
        a_scales, a_values = split_ggml_q8_0_blocks(xq)
        y = torch.empty((rows, n), dtype=torch.float32, device="cuda")
        y_split = torch.empty((rows, n), dtype=torch.float32, device="cuda")
        runner = Runner(torch, torch.cuda.Stream())
        runner.uses(xq, wq, y, a_values, a_scales, w_words, w_scales, y_split)
        runner.add("qxt_ggml_q4_0_q8_0_linear", _p(xq), _rs(xq), _p(wq), _rs(wq), _p(y), _rs(y),
                   rows, k // 32, 0, 0, n, runner.handle)
        runner.add("qxt_ggml_q4_0_q8_0_tiled_linear", _p(a_values), _rs(a_values), _p(a_scales), _rs(a_scales),
                   a_scales.element_size(), _p(w_words), _rs(w_words), _p(w_scales), _rs(w_scales), _p(y_split),
                   _rs(y_split), rows, k // 32, n, runner.handle)
        runner.run()
        torch.cuda.synchronize()
        times = runner.kernel_times(repeats=5)["q4_0_tiled_kernel"]
        native_us = float(np.mean(times[0::2])) * 1e3
        split_us = float(np.mean(times[1::2])) * 1e3
        if not torch.equal(y, y_split):
            raise RuntimeError("prefill: native and split layouts disagree")
        valu_ops = rows * n * (k // 32) * 4
        best = min(native_us, split_us)
        out[label] = {
            "shape": f"M={rows} K={k} N={n}",
            "kernel_us": best,
            "layout": "split" if split_us <= native_us else "native",
            "native_kernel_us": native_us,
            "split_kernel_us": split_us,
            "tops": 2 * rows * n * k / (best * 1e-6) / 1e12,
            "valu_bound_us": valu_ops / valu_peak * 1e6,
            "frac_valu_bound": valu_ops / valu_peak / (best * 1e-6),
            "check": check_q4_0(torch, f"prefill {label}", q8_0_host(torch, x[[0, rows - 1]]), wq,
                                y[[0, rows - 1]], rows=(0, 1)),
        }
        del wq, x, xq, y, y_split, w_scales, w_words, a_scales, a_values
        torch.cuda.synchronize()
    return out


def leg_geglu(torch, args) -> dict:
    """GEGLU -> Q8_0 producer at the FFN width 5632: M = 1 (decode), 512 and 2048 (prefill).

    HBM-bound: per 32-element block it reads 256 B of fp32 gate + up and
    writes one 34-byte Q8_0 block (290 algorithmic bytes); the 128 KB GELU
    table is read through the caches.  Launches rotate over enough buffer
    sets (> 320 MB) that every launch reads its inputs from HBM, not from the
    256 MB last-level cache.
    """
    from qpu_xla_amd.kernels.ggml_geglu_q8 import ggml_gelu_fp16_table

    gen = torch.Generator(device="cuda")
    gen.manual_seed(7)
    table = ggml_gelu_fp16_table("cuda")
    k = 5632
    out = {}
    for rows in (1, 512, 2048):
        nsets = min(64, max(2, -(-(320 << 20) // (rows * k * 8))))
        sets = [
            (torch.randn((rows, k), generator=gen, device="cuda"), torch.randn((rows, k), generator=gen, device="cuda"),
             torch.empty((rows, k // 32, 34), dtype=torch.uint8, device="cuda"))
            for _ in range(nsets)
        ]
        runner = Runner(torch, torch.cuda.Stream())
        for gate, up, q8 in sets:
            runner.uses(gate, up, q8)
            runner.add("qxt_ggml_geglu_q8_0", _p(gate), _rs(gate), _p(up), _rs(up), _p(table), _p(q8), _rs(q8),
                       rows, k, runner.handle)
        runner.run()
        torch.cuda.synchronize()
        times = runner.kernel_times(repeats=max(1, 64 // nsets))
        us = float(np.mean(next(v for name, v in times.items() if name.startswith("geglu_q8_0")))) * 1e3
        nbytes = rows * (k // 32) * (256 + 34)
        out[f"m{rows}"] = {
            "shape": f"M={rows} K={k}",
            "buffer_sets": nsets,
            "kernel_us": us,
            "bytes_per_launch": nbytes,
            "gbs": nbytes / (us * 1e-6) / 1e9,
            "frac_hbm_peak": nbytes / (us * 1e-6) / 1e9 / PEAK_HBM_GBS,
        }
        # Last launch: v = fl32(table[fp16(gate)] * up), then the Q8_0 rule, on row 0.
        torch.cuda.synchronize()
        gate, up, q8 = sets[-1]
        index = gate[0].cpu().half().view(torch.int16).to(torch.int64) & 0xFFFF
        gelu = table.cpu().view(torch.int16)[index].view(torch.float16).float()
        want = q8_0_host(torch, (gelu * up[0].cpu())[None])
        if not torch.equal(q8[0].cpu(), want[0]):
            raise RuntimeError(f"geglu M={rows}: row 0 differs from the reference arithmetic")
        out[f"m{rows}"]["check"] = {"rows_checked": [0], "blocks": k // 32, "bit_exact": True}
        del sets
        torch.cuda.empty_cache()
    return out


def leg_cfg1(torch, args) -> dict:
    """cfg1: W8A8 M=K=N=512 whole operator (launch-bound; parity case, reported only)."""
    gen = torch.Generator(device="cuda")
    gen.manual_seed(1)
    m = k = n = 512
    x = torch.randn((m, k), generator=gen, device="cuda", dtype=torch.float32)
    from qpu_xla_amd.quantization import quantize_per_output_channel_int8

    weight = quantize_per_output_channel_int8(torch.randn((n, k), generator=gen, device="cuda") * 0.05)
    bias = torch.randn((n,), generator=gen, device="cuda") * 0.1
    qa = torch.empty((m, k), dtype=torch.int8, device="cuda")
    sa = torch.empty((m,), dtype=torch.float32, device="cuda")
    y = torch.empty((m, n), dtype=torch.float32, device="cuda")
    runner = Runner(torch, torch.cuda.Stream())
    for _ in range(32):
        runner.add("qxt_w8a8_linear", _p(x), _rs(x), _p(qa), _rs(qa), _p(sa), _p(weight.values), _rs(weight.values),
                   _p(weight.scales), _p(bias), _p(y), _rs(y), m, n, k, 0, 0, runner.handle)
    runner.run()
    times = runner.kernel_times()
    graph = runner.capture()
    wall_ms, _ = runner.timed_graph(graph, 10, 2)
    torch.cuda.synchronize()
    check = check_w8a8(torch, "cfg1", x, qa, sa, weight, bias, y, rows=(0, m - 1))
    return {
        "check": check,
        "shape": "M=K=N=512",
        "operator_us": wall_ms * 1e3 / 32,
        "gemm_kernel_us": gemm_kernel_ms(times) * 1e3 / 32,
        "quantise_kernel_us": float(np.sum(times["rows_int8_kernel"])) * 1e3 / 32,
        "operator_tops": 2 * m * n * k / (wall_ms * 1e-3 / 32) / 1e12,
    }


def leg_copy(torch) -> dict:
    """Device-to-device copy ceiling (reads + writes) and the plain streaming read rate
    (``qxt_hbm_read_probe`` over 1 GiB), for context next to the 8 TB/s spec."""
    nbytes = 1 << 30
    src = torch.empty(nbytes // 4, dtype=torch.float32, device="cuda").fill_(1.0)
    dst = torch.empty_like(src)
    for _ in range(3):
        dst.copy_(src)
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(10):
        dst.copy_(src)
    end.record()
    torch.cuda.synchronize()
    ms = start.elapsed_time(end) / 10
    del dst
    # Read ceiling: the library's plain streaming read of the same 1 GiB.
    from qpu_xla_amd import _lib

    partials = torch.empty(2048, dtype=torch.int32, device="cuda")
    stream = ctypes.c_void_p(int(torch.cuda.current_stream().cuda_stream))
    for _ in range(3):
        _lib.call("qxt_hbm_read_probe", _p(src), nbytes, _p(partials), stream)
    torch.cuda.synchronize()
    start.record()
    for _ in range(10):
        _lib.call("qxt_hbm_read_probe", _p(src), nbytes, _p(partials), stream)
    end.record()
    torch.cuda.synchronize()
    read_ms = start.elapsed_time(end) / 10
    del src, partials
    torch.cuda.empty_cache()
    return {"bytes": 2 * nbytes, "gbs": 2 * nbytes / (ms * 1e-3) / 1e9,
            "read_bytes": nbytes, "read_gbs": nbytes / (read_ms * 1e-3) / 1e9}


def cpu_baseline_q4(budget_s: float) -> dict:
    """The NumPy oracle (reference CPU path) on the cfg3 decode step, bounded by ``budget_s``.

    Weights are prepared once (outside the timed region); the timed work is
    Q8_0 quantisation + the Q4_0 x Q8_0 oracle of every linear, whole steps
    repeated until the budget is spent.
    """
    import oracle

    rng = np.random.default_rng(3)
    linears = []
    for _ in range(LAYERS):
        for (_, k, n) in TINYLLAMA_LAYER:
            w = (rng.standard_normal((n, k), dtype=np.float32) * np.float32(0.02)).astype(np.float32)
            linears.append((oracle.quantize_q4_0_blocks(w), rng.standard_normal((1, k), dtype=np.float32), k, n))
    step_bytes = sum(q4_linear_bytes(1, k, n) for (_, _, k, n) in linears)
    steps = 0
    t0 = time.perf_counter()
    while True:
        for wq, x, _, _ in linears:
            xq = oracle.quantize_q8_0_blocks(x)
            oracle.q4_0_q8_0_reference(xq, wq)
        steps += 1
        elapsed = time.perf_counter() - t0
        if elapsed >= budget_s:
            break
    return {
        "value": steps * step_bytes / elapsed / 1e9,
        "unit": "GB/s",
        "cores": 1,
        "kind": "port",
        "sample": f"{steps} whole cfg3 decode steps (154 linears: Q8_0 quantise + Q4_0xQ8_0 oracle, NumPy, "
        f"single thread), {steps * step_bytes / 1e6:.1f} MB in {elapsed:.2f} s",
    }


def cpu_baseline_w8a8(budget_s: float) -> dict:
    """NumPy oracle of the dynamic W8A8 linear on a row sample of cfg4 gate/up (int32 matmul is not BLAS)."""
    import oracle

    rng = np.random.default_rng(4)
    k, n = 4096, 14336
    w = (rng.standard_normal((n, k), dtype=np.float32) * np.float32(0.02)).astype(np.float32)
    qw, sw = oracle.quantize_per_output_channel_int8(w)
    qw32 = qw.astype(np.int32)
    bias = (rng.standard_normal(n, dtype=np.float32) * np.float32(0.1)).astype(np.float32)
    rows = 0
    elapsed = 0.0
    while elapsed < budget_s and rows < 1024:
        x = rng.standard_normal((8, k), dtype=np.float32)
        t0 = time.perf_counter()
        qa, sa = oracle.quantize_rows_int8(x)
        acc = qa.astype(np.int32) @ qw32.T
        oracle.dequantize_epilogue(acc, sa, sw, bias)
        elapsed += time.perf_counter() - t0
        rows += 8
    return {
        "value": 2 * rows * n * k / elapsed / 1e12,
        "unit": "TOPS",
        "cores": 1,
        "kind": "port",
        "sample": f"{rows} of 4096 rows of cfg4 gate/up (K=4096, N=14336), NumPy int32 matmul, {elapsed:.2f} s",
    }


def _blas_threads() -> int | None:
    """Threads of NumPy's BLAS (threadpoolctl), or None when it cannot tell."""
    try:
        from threadpoolctl import threadpool_info
    except ImportError:
        return None
    counts = [pool.get("num_threads") for pool in threadpool_info() if pool.get("user_api") == "blas"]
    return max(counts) if counts else None


def cpu_references_w8a8(budget_s: float) -> dict:
    """The reference benchmark's other CPU references on a row sample of cfg4 gate/up.

    examples/benchmark_qpu_xla_w8a8.py:199-265: the dynamic W8A8 projection in
    torch int32 (per-row activation quantisation, int32 matmul, fp32
    scaling), and the unquantised fp32 projection in NumPy (BLAS) and torch.
    Each is timed with 2 warm-up calls and up to 7 timed calls within its
    share of ``budget_s``; ``threads`` is what the library used.
    """
    import oracle
    import torch

    rng = np.random.default_rng(4)
    k, n = 4096, 14336
    w = (rng.standard_normal((n, k), dtype=np.float32) * np.float32(0.02)).astype(np.float32)
    qw, sw = oracle.quantize_per_output_channel_int8(w)
    torch_w32 = torch.from_numpy(qw.astype(np.int32))
    torch_sw = torch.from_numpy(sw)
    torch_w = torch.from_numpy(w)

    def torch_int32(x):
        t = torch.from_numpy(x)
        sa = torch.maximum(torch.amax(torch.abs(t), dim=1) / 127, torch.tensor(1.0 / 127.0))
        q = torch.round(t / sa[:, None]).clamp(-127, 127).to(torch.int32)
        return (q @ torch_w32.T).to(torch.float32) * sa[:, None] * torch_sw[None, :]

    cases = {
        "torch_int32_w8a8": (16, torch_int32),
        "numpy_fp32": (64, lambda x: x @ w.T),
        "torch_fp32": (64, lambda x: torch.from_numpy(x) @ torch_w.T),
    }
    out = {}
    for name, (rows, fn) in cases.items():
        x = rng.standard_normal((rows, k), dtype=np.float32)
        for _ in range(2):
            fn(x)
        times = []
        t_start = time.perf_counter()
        while len(times) < 7 and time.perf_counter() - t_start < budget_s / len(cases):
            t0 = time.perf_counter()
            fn(x)
            times.append(time.perf_counter() - t0)
        best = min(times)
        out[name] = {
            "value": 2 * rows * n * k / best / 1e12,
            "unit": "TOPS",
            "rows": rows,
            "shape": f"M={rows} K={k} N={n}",
            "calls": len(times),
            "best_ms": best * 1e3,
            "threads": torch.get_num_threads() if name.startswith("torch") else _blas_threads(),
        }
    return out


def measured_traffic(kernel: str) -> dict | None:
    """HBM bytes per launch of `kernel` from the committed rocprofv3 FETCH/WRITE summary, if any."""
    path = ROOT / "profiles" / f"{kernel}_cfg3_traffic.json"
    try:
        with open(path) as fh:
            data = json.load(fh)
    except (OSError, ValueError):
        return None
    if data.get("kernel") != kernel:
        return None
    return {"bytes": int(data["hbm_bytes_per_launch"]), "source": str(path.relative_to(ROOT))}


def host_info() -> dict:
    info = {"cpu_count": os.cpu_count()}
    try:
        info["affinity"] = len(os.sched_getaffinity(0))
    except AttributeError:
        pass
    for var in ("OMP_NUM_THREADS", "OPENBLAS_NUM_THREADS"):
        info[var] = os.environ.get(var)
    try:
        import torch

        info["torch_threads"] = torch.get_num_threads()
    except ImportError:
        pass
    try:
        blas = np.show_config(mode="dicts").get("Build Dependencies", {}).get("blas", {})
        info["numpy_blas"] = f"{blas.get('name')} {blas.get('version')}"
    except (TypeError, AttributeError):
        pass
    try:
        with open("/proc/cpuinfo") as fh:
            for line in fh:
                if line.startswith("model name"):
                    info["cpu_model"] = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    return info


def main() -> int:
    args = parse_args()
    if args.gpus != 1:
        print(
            "bench.py measures one GPU only: the quantized-linear path is benchmarked per device "
            "(multi-GPU sharding is a design note, not a measured configuration); run with --gpus 1",
            file=sys.stderr,
        )
        return 2
    import torch

    if not torch.cuda.is_available():
        print("bench.py needs a HIP device", file=sys.stderr)
        return 1
    from qpu_xla_amd import _lib

    info = _lib.device_info()
    legs = set(args.legs.split(","))
    device = {
        "arch": info.arch.decode(),
        "compute_units": info.compute_units,
        "clock_mhz": info.clock_khz / 1e3,
        "hbm_gib": info.total_memory / 2**30,
    }
    log(f"device {device}")
    out: dict = {}
    if "decode" in legs:
        log("leg decode (cfg3)")
        out["decode"] = leg_decode(torch, args)
        log(f"decode: {out['decode']}")
    if "cfg0" in legs:
        log("leg cfg0 rotated")
        out["cfg0"] = leg_rotated_q4(torch, args, 1, 2048, 5632, 0)
        log(f"cfg0: {out['cfg0']}")
    if "cfg2" in legs:
        log("leg cfg2 rotated")
        out["cfg2"] = [leg_rotated_q4(torch, args, 4, 4096, 11008, 2), leg_rotated_q4(torch, args, 4, 4096, 4096, 2)]
        # The same launches over the native ggml rows (the drop-in layout, no re-layout).
        out["cfg2_native_layout"] = [leg_rotated_q4(torch, args, 4, 4096, 11008, 2, "native"),
                                     leg_rotated_q4(torch, args, 4, 4096, 4096, 2, "native")]
        log(f"cfg2: {out['cfg2']}")
    if "q4_long" in legs:
        log("leg q4_0 long rows (native layout)")
        out["q4_0_long_rows"] = [leg_rotated_q4(torch, args, m, k, n, 8, "native")
                                 for m, k, n in ((2, 5632, 2048), (4, 5632, 2048), (1, 11008, 4096),
                                                 (4, 11008, 4096), (4, 14336, 4096))]
        log(f"q4_0 long rows: {out['q4_0_long_rows']}")
    if "q8_0" in legs:
        log("leg q8_0 x q8_0 rotated")
        out["q8_0_q8_0"] = [leg_rotated_q8(torch, args, 1, 2048, 5632, 7), leg_rotated_q8(torch, args, 4, 4096, 11008, 7),
                            leg_rotated_q8(torch, args, 4, 4096, 4096, 7)]
        log(f"q8_0 x q8_0: {out['q8_0_q8_0']}")
    if "w8a8" in legs:
        log("leg w8a8 (cfg4)")
        out["w8a8"] = leg_w8a8(torch, args)
        log(f"w8a8: {out['w8a8']}")
    if "gemv" in legs:
        log("leg w8a8 gemv (M=1)")
        out["gemv"] = leg_w8a8_gemv(torch, args)
        log(f"gemv: {out['gemv']}")
    if "prefill" in legs:
        log("leg q4_0 prefill (M=512)")
        out["prefill"] = leg_prefill(torch, args)
        log(f"prefill: {out['prefill']}")
    if "geglu" in legs:
        log("leg geglu -> q8_0 producer")
        out["geglu"] = leg_geglu(torch, args)
        log(f"geglu: {out['geglu']}")
    if "shards" in legs:
        log("leg shards (one GPU's share of an 8-GPU sharding)")
        out["shards"] = leg_shards(torch, args)
        log(f"shards: {out['shards']}")
    if "cfg1" in legs:
        log("leg cfg1")
        out["cfg1"] = leg_cfg1(torch, args)
        log(f"cfg1: {out['cfg1']}")
    if "copy" in legs:
        out["copy"] = leg_copy(torch)
        log(f"copy: {out['copy']}")
    cpu = None
    cpu_w8a8 = None
    if "cpu" in legs:
        log("cpu baseline (NumPy oracle)")
        cpu = cpu_baseline_q4(args.cpu_seconds)
        cpu_w8a8 = cpu_baseline_w8a8(args.cpu_seconds)
        cpu_w8a8["reference_cpu_paths"] = cpu_references_w8a8(args.cpu_seconds)
        cpu["host"] = host_info()
        log(f"cpu: {cpu} / {cpu_w8a8}")

    decode = out.get("decode")
    head = decode["batched"] if decode else None
    traffic = measured_traffic("q4_0_batch_kernel")
    line = {
        "metric": METRIC,
        "value": head["gbs"] if head else None,
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": head["ms_per_step_wall"] if head else None,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8 dot4 (Q4_0 x Q8_0) -> int32 block dots -> fp32",
        "data": "synthetic (seeded N(0,0.02) weights quantised to Q4_0, N(0,1) activations)",
        "config": {
            "workload": "cfg3: TinyLlama-1.1B decode step, 22 layers x 7 Q4_0xQ8_0 linears "
            "(q/o 2048x2048, k/v 2048->256, gate/up 2048->5632, down 5632->2048), M=1, "
            "Q8_0 re-quantisation of each linear's activation (one pre-pass launch for all 154), then all 154 "
            "linears in one batched launch per step",
            "bytes_per_step": decode["bytes_per_step"] if decode else None,
            "frac_hbm_peak": head["gbs"] / PEAK_HBM_GBS if head else None,
            "schedule": "batched",
        },
        "roofline": (
            {
                "bound": "hbm",
                "kernel": "q4_0_batch_kernel",
                "achieved": head["kernel_gbs"],
                "peak": PEAK_HBM_GBS,
                "unit": "GB/s",
                "frac": head["kernel_gbs"] / PEAK_HBM_GBS,
                "frac_of_measured_read_rate": (head["kernel_gbs"] / out["copy"]["read_gbs"]
                                               if out.get("copy", {}).get("read_gbs") else None),
                "traffic": (traffic or {}).get("bytes"),
                "traffic_source": (traffic or {}).get("source"),
                "bytes_per_launch": head["kernel_bytes_per_launch"],
                "avg_launch_us": head["kernel_avg_us"],
            }
            if head
            else None
        ),
        "cpu_baseline": cpu,
        "w8a8": out.get("w8a8"),
        "w8a8_gemv": out.get("gemv"),
        "q4_0_prefill": out.get("prefill"),
        "geglu_q8_0": out.get("geglu"),
        "q8_0_q8_0": out.get("q8_0_q8_0"),
        "q4_0_long_rows": out.get("q4_0_long_rows"),
        "shards": out.get("shards"),
        "w8a8_cpu_baseline": cpu_w8a8,
        "decode": decode,
        "configs": {key: out[key] for key in ("cfg0", "cfg1", "cfg2", "cfg2_native_layout") if key in out},
        "copy_ceiling_gbs": out.get("copy", {}).get("gbs"),
        "read_ceiling_gbs": out.get("copy", {}).get("read_gbs"),
        "device": device,
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
