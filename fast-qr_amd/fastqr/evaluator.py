"""The task evaluator's benchmark loop, as a reusable harness.

Restates official/eval.py:96-110 (``calculate_stats``), 157-175 (inputs per
timed repeat, seed += 42 before each), 178-224 (``_run_single_benchmark``:
pre-timing check, cache flush and device-event timing per repeat, recheck,
adaptive stopping) and 227-251 (``run_benchmarking``: one warm-up case, then
every case with recheck on).  The device-specific pieces (the kernel, the
input generator, the checker, the cache flush and the timer) are arguments,
so the loop itself runs, and is tested, without a GPU.

Deviations from the evaluator, chosen by the caller and reported with the
results: ``recheck="bitwise"`` compares every timed output with the checked
pre-timing output bit for bit instead of re-running the checker on it (the
kernels are deterministic; the CPU checker would dominate the wall time of the
large cases), and ``check_matrices`` limits the pre-timing check to the first
k matrices of every input.
"""
from __future__ import annotations

import math
import time
from dataclasses import dataclass, replace
from typing import Any, Callable, Sequence

# official/eval.py: MAX_ITERATIONS_PER_BENCHMARK, BENCHMARK_INPUT_BYTES_TARGET
MAX_INPUTS_PER_REPEAT = 50
INPUT_BYTES_TARGET = 256 * 1024 * 1024
SEED_STEP = 42
# official/eval.py:214-222 and 228, 246
MIN_ELAPSED_NS = 1e8
REL_ERR_STOP = 0.001
HARD_LIMIT_NS = 120e9
WARMUP_MAX_TIME_NS = 1e8
BENCH_MAX_TIME_NS = 10e9
MAX_REPEATS = 200


@dataclass(frozen=True)
class Stats:
    """official/eval.py Stats: durations in ns per kernel call."""
    runs: int
    mean: float
    std: float
    err: float
    best: float
    worst: float


def calculate_stats(durations: Sequence[float]) -> Stats:
    """official/eval.py:96-110: sample std (n - 1), err = std / sqrt(runs)."""
    runs = len(durations)
    avg = sum(durations) / runs
    var = sum((x - avg) ** 2 for x in durations)
    std = math.sqrt(var / (runs - 1)) if runs > 1 else 0.0
    err = std / math.sqrt(runs) if runs > 0 else 0.0
    return Stats(runs, avg, std, err, float(min(durations)), float(max(durations)))


def inputs_per_repeat(batch: int, n: int) -> int:
    """official/eval.py:167-175: inputs timed per repeat (fp32 A only)."""
    per_input = 4 * batch * n * n
    if per_input <= 0:
        return 1
    return max(1, min(MAX_INPUTS_PER_REPEAT, INPUT_BYTES_TARGET // per_input))


def input_seeds(seed: int, count: int) -> list[int]:
    """official/eval.py:157-164: the seed advances by 42 before every input."""
    return [seed + SEED_STEP * (i + 1) for i in range(count)]


def should_stop(i: int, durations: Sequence[float], elapsed_ns: float, max_time_ns: float) -> bool:
    """official/eval.py:214-222: after repeat i (0-based), once more than two
    repeats and 0.1 s have passed, stop when the standard error falls below
    0.1% of the mean, the summed kernel time exceeds max_time_ns, or 120 s of
    wall time have gone by."""
    if i <= 1 or elapsed_ns <= MIN_ELAPSED_NS:
        return False
    st = calculate_stats(durations)
    return st.err / st.mean < REL_ERR_STOP or st.mean * st.runs > max_time_ns or elapsed_ns > HARD_LIMIT_NS


@dataclass
class Device:
    """What the loop needs from the device.

    kernel(data) -> output; clone(data) -> an independent copy;
    check(data, output) -> (ok, message), the task's checker;
    flush() clears the caches before a repeat; sync() waits for the device;
    time_calls(fn) -> (outputs, elapsed ns) runs fn() between device events;
    same(out_a, out_b) -> bool, bitwise equality of two outputs.
    """
    kernel: Callable[[Any], Any]
    clone: Callable[[Any], Any]
    check: Callable[[Any, Any], tuple]
    flush: Callable[[], None]
    sync: Callable[[], None]
    time_calls: Callable[[Callable[[], list]], tuple]
    same: Callable[[Any, Any], bool]
    clock_ns: Callable[[], int] = time.perf_counter_ns


def run_single_benchmark(spec, generate: Callable[[Any], Any], dev: Device, recheck: str | None,
                         max_repeats: int, max_time_ns: float, check_matrices: int | None = None):
    """official/eval.py:178-224.  Returns Stats, or the failure message.

    ``spec`` is a dataclass with ``batch``, ``n`` and ``seed`` (fastqr.cases.Case);
    ``generate(spec)`` builds one input.  ``recheck`` is None (no recheck),
    "checker" (the checker on every timed output, as the evaluator) or
    "bitwise" (every timed output equal to the checked one)."""
    count = inputs_per_repeat(spec.batch, spec.n)
    data_list = [generate(replace(spec, seed=s)) for s in input_seeds(spec.seed, count)]
    check_copy = [dev.clone(d) for d in data_list]
    outputs = [dev.kernel(dev.clone(d)) for d in data_list]
    dev.sync()
    checked = []
    for ref, out in zip(check_copy, outputs):
        good, message = _check(dev, ref, out, check_matrices)
        if not good:
            return message
        checked.append(tuple(dev.clone(o) for o in out))
    durations = []
    start = dev.clock_ns()
    for i in range(max_repeats):
        dev.sync()
        dev.flush()
        outs, elapsed_ns = dev.time_calls(lambda: [dev.kernel(d) for d in data_list])
        dev.sync()
        durations.append(elapsed_ns / len(data_list))
        if recheck == "checker":
            for ref, out in zip(check_copy, outs):
                good, message = _check(dev, ref, out, check_matrices)
                if not good:
                    return message
        elif recheck == "bitwise":
            for out, ref_out in zip(outs, checked):
                if not dev.same(out, ref_out):
                    return "a timed output differs from the checked pre-timing output"
        if should_stop(i, durations, dev.clock_ns() - start, max_time_ns):
            break
    return calculate_stats(durations)


def _check(dev: Device, data, output, check_matrices):
    if check_matrices is None:
        return dev.check(data, output)
    k = check_matrices
    return dev.check(data[:k], tuple(o[:k] for o in output))


def run_benchmarking(specs: Sequence, generate: Callable[[Any], Any], dev: Device, recheck: str = "bitwise",
                     check_matrices: int | None = None, max_repeats: int = MAX_REPEATS,
                     max_time_ns: float = BENCH_MAX_TIME_NS, warmup_max_time_ns: float = WARMUP_MAX_TIME_NS,
                     on_result: Callable[[int, Any, Any], None] | None = None):
    """official/eval.py:227-251: a warm-up run of the first case (no recheck),
    then every case.  Returns (results, passed); results[i] is Stats or the
    failure message of case i."""
    run_single_benchmark(specs[0], generate, dev, None, max_repeats, warmup_max_time_ns, check_matrices)
    results, passed = [], True
    for idx, spec in enumerate(specs):
        res = run_single_benchmark(spec, generate, dev, recheck, max_repeats, max_time_ns, check_matrices)
        if not isinstance(res, Stats):
            passed = False
        results.append(res)
        if on_result is not None:
            on_result(idx, spec, res)
    return results, passed


def torch_device(torch_mod, kernel, check, flush_bytes: int = 1 << 30, device: str = "cuda:0") -> Device:
    """A Device on a torch GPU: HIP events around the timed calls on torch's
    current stream, a flush buffer of ``flush_bytes`` (1 GiB: MI355X has a
    256 MB Infinity Cache; the evaluator writes 256 MiB).  ``check(a, h, tau)``
    is the task's checker on CPU tensors."""
    buf = torch_mod.empty(flush_bytes // 8, dtype=torch_mod.int64, device=device)

    def time_calls(fn):
        e0 = torch_mod.cuda.Event(enable_timing=True)
        e1 = torch_mod.cuda.Event(enable_timing=True)
        e0.record()
        outs = fn()
        e1.record()
        torch_mod.cuda.synchronize()
        return outs, e0.elapsed_time(e1) * 1e6

    def clone(x):
        return x.clone()

    def same(a, b):
        return all(torch_mod.equal(x, y) for x, y in zip(a, b))

    def check_on_cpu(data, out):
        return check(data.cpu(), *(o.cpu() for o in out))

    return Device(kernel=kernel, clone=clone, check=check_on_cpu, flush=lambda: buf.fill_(42),
                  sync=torch_mod.cuda.synchronize, time_calls=time_calls, same=same)
