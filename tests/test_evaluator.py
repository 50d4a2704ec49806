"""The evaluator's benchmark loop (fastqr.evaluator, restating
official/eval.py:96-110, 157-251) driven without a GPU: closed-form statistics,
the inputs-per-repeat and seed rules, the adaptive stopping rule, and whole
runs on a scripted device with a fake clock (CPU tensors, a toy kernel)."""
import math
from dataclasses import dataclass

import pytest
import torch

from fastqr import evaluator
from fastqr.cases import BENCHMARKS, Case


def test_stats_closed_form():
    st = evaluator.calculate_stats([1.0, 2.0, 3.0, 4.0])
    assert st.runs == 4 and st.mean == 2.5 and st.best == 1.0 and st.worst == 4.0
    assert math.isclose(st.std, math.sqrt(5.0 / 3.0))  # sample variance, n - 1
    assert math.isclose(st.err, math.sqrt(5.0 / 3.0) / 2.0)
    one = evaluator.calculate_stats([7.0])
    assert one.std == 0.0 and one.err == 0.0


def test_inputs_per_repeat_matches_the_evaluator_counts():
    # 256 MiB of fp32 A per repeat, clamped to [1, 50] (official/eval.py:167-175)
    counts = {(c.batch, c.n): evaluator.inputs_per_repeat(c.batch, c.n) for c in BENCHMARKS}
    assert counts == {(20, 32): 50, (40, 176): 50, (40, 352): 13, (640, 512): 1, (60, 1024): 1,
                      (8, 2048): 2, (2, 4096): 2}
    assert evaluator.inputs_per_repeat(0, 5) == 1


def test_seed_advances_by_42_before_every_input():
    assert evaluator.input_seeds(100, 3) == [142, 184, 226]


def test_stopping_rule():
    flat = [10.0] * 5
    assert not evaluator.should_stop(1, flat[:2], 5e8, 1e10)  # never before the third repeat
    assert not evaluator.should_stop(4, flat, 0.9e8, 1e10)  # nor before 0.1 s of wall time
    assert evaluator.should_stop(4, flat, 2e8, 1e10)  # zero spread: err / mean < 0.001
    noisy = [1.0, 100.0, 1.0, 100.0, 1.0]
    assert not evaluator.should_stop(4, noisy, 2e8, 1e10)
    assert evaluator.should_stop(4, noisy, 2e8, 200.0)  # summed kernel time above the budget
    assert evaluator.should_stop(4, noisy, 121e9, 1e10)  # 120 s of wall time


@dataclass
class Script:
    """A scripted device: per timed repeat, a duration and a clock advance."""
    durations: list
    clock_step_ns: float = 5e7
    corrupt_at: int | None = None  # timed repeat whose outputs differ
    fail_check: bool = False

    def device(self):
        state = {"t": 0, "repeat": 0, "generated": []}

        def kernel(x):
            out = (x * 2.0, x.sum(dim=-1))
            if state.get("timing") and self.corrupt_at == state["repeat"]:
                out = (out[0] + 1.0, out[1])
            return out

        def time_calls(fn):
            state["timing"] = True
            outs = fn()
            state["timing"] = False
            d = self.durations[min(state["repeat"], len(self.durations) - 1)]
            state["repeat"] += 1
            state["t"] += self.clock_step_ns
            return outs, d * len(outs)

        def check(data, out):
            if self.fail_check:
                return False, "checker says no"
            return bool(torch.equal(out[0], data * 2.0)), "ok"

        dev = evaluator.Device(kernel=kernel, clone=lambda x: x.clone(), check=check, flush=lambda: None,
                               sync=lambda: None, time_calls=time_calls,
                               same=lambda a, b: all(torch.equal(x, y) for x, y in zip(a, b)),
                               clock_ns=lambda: state["t"])
        return dev, state


def _generate(seen):
    def gen(c):
        seen.append(c.seed)
        return torch.full((c.batch, 2, 2), float(c.seed))
    return gen


def test_run_single_benchmark_stops_on_a_flat_series():
    dev, state = Script([1000.0]).device()
    seen = []
    st = evaluator.run_single_benchmark(Case(20, 32, 1, 7), _generate(seen), dev, "bitwise", 200, 10e9)
    assert isinstance(st, evaluator.Stats)
    # the clock passes 0.1 s after the third repeat (5e7 ns each): the first
    # check that may stop is after repeat i = 2 at 1.5e8 ns
    assert st.runs == 3 and st.mean == 1000.0
    assert seen == evaluator.input_seeds(7, 50)  # 20 x 32: 50 inputs per repeat
    assert state["repeat"] == 3


def test_run_single_benchmark_runs_to_the_cap_on_a_noisy_series():
    dev, _ = Script([1.0, 1000.0] * 10).device()
    st = evaluator.run_single_benchmark(Case(2, 4096, 1, 1), _generate([]), dev, "checker", 20, 10e9)
    assert st.runs == 20


def test_recheck_catches_a_timed_output_that_differs():
    dev, _ = Script([1000.0, 2000.0], corrupt_at=1).device()
    res = evaluator.run_single_benchmark(Case(8, 2048, 1, 3), _generate([]), dev, "bitwise", 200, 10e9)
    assert isinstance(res, str) and "differs" in res
    dev, _ = Script([1000.0, 2000.0], corrupt_at=1).device()
    res = evaluator.run_single_benchmark(Case(8, 2048, 1, 3), _generate([]), dev, "checker", 200, 10e9)
    assert res == "ok"  # the checker's message for the failing output


def test_pre_timing_check_failure_is_reported():
    dev, state = Script([1000.0], fail_check=True).device()
    res = evaluator.run_single_benchmark(Case(8, 2048, 1, 3), _generate([]), dev, "bitwise", 200, 10e9)
    assert res == "checker says no" and state["repeat"] == 0


def test_run_benchmarking_two_cases():
    dev, state = Script([500.0]).device()
    seen = []
    specs = [Case(20, 32, 1, 10), Case(2, 4096, 1, 20)]
    got = []
    results, passed = evaluator.run_benchmarking(specs, _generate(seen), dev,
                                                 on_result=lambda i, c, r: got.append((i, c, r)))
    assert passed and len(results) == 2 and all(isinstance(r, evaluator.Stats) for r in results)
    # a warm-up run of the first case, then both cases
    assert seen[:50] == evaluator.input_seeds(10, 50) and seen[50:100] == evaluator.input_seeds(10, 50)
    assert seen[100:] == evaluator.input_seeds(20, 2)
    assert [i for i, _, _ in got] == [0, 1]


def test_run_benchmarking_reports_a_failing_case():
    dev, _ = Script([500.0], corrupt_at=4).device()
    specs = [Case(20, 32, 1, 10), Case(2, 4096, 1, 20)]
    results, passed = evaluator.run_benchmarking(specs, _generate([]), dev)
    # the warm-up (repeats 0-2) has no recheck; the first case's repeat 4 differs
    assert not passed and isinstance(results[0], str) and isinstance(results[1], evaluator.Stats)


@pytest.mark.parametrize("bad", [0, -1])
def test_inputs_per_repeat_degenerate(bad):
    assert evaluator.inputs_per_repeat(bad, 8) == 1


def test_torch_device_adapts_the_task_checker():
    # Device.check(data, output) calls the task's checker as check(a, h, tau)
    from oracle import checker

    dev = evaluator.torch_device(torch, kernel=None, check=checker.official_check, flush_bytes=64, device="cpu")
    a = torch.randn((2, 8, 8), generator=torch.Generator().manual_seed(3))
    ok, msg = dev.check(a, torch.geqrf(a))
    assert ok, msg
    h, tau = torch.geqrf(a)
    ok, _ = dev.check(a, (h, tau * 1.5))
    assert not ok
    assert dev.same((h, tau), (h.clone(), tau.clone())) and not dev.same((h, tau), (h, tau + 1))
