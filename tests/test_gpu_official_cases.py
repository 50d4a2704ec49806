"""GPU parity on the official task's 22 test cases (official/task.yml:85-107):
every conditioning profile and the mixed batches, inputs from the restated
generator (fastqr.cases, drawn on the CPU), factored by the HIP path and
checked against the oracle (CPU torch.geqrf) with the evaluator's checker
(official/reference.py:182-266) and this build's stated tolerances.
"""
import sys

import pytest
import torch

from fastqr import cases, custom_kernel
from oracle import checker

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("case", cases.TESTS, ids=[c.label for c in cases.TESTS])
def test_official_case(cuda, case):
    print(f"[official] {case.label}", flush=True)
    sys.stdout.flush()
    a = cases.generate(case)
    h, tau = custom_kernel(a.to(cuda))
    torch.cuda.synchronize()
    h, tau = h.cpu(), tau.cpu()
    ok, msg = checker.official_check(a, h, tau)
    assert ok, msg
    rep = checker.frobenius_gates(a, h, tau)
    assert rep.ok, rep.message()
    h_ref, tau_ref = torch.geqrf(a)
    ag = checker.rdiag_tau_agreement(a, h, tau, h_ref, tau_ref)
    assert ag.ok, ag.message()
    if case.case == "upper":
        # an upper-triangular input has nothing to annihilate: tau == 0, H == A
        assert torch.count_nonzero(tau) == 0
        assert torch.equal(h, a)
    print(f"  {msg}; {ag.message()}", flush=True)


def stratified_sample(labels, per_family=3):
    """First and last matrix, both sides of the first and last 8-matrix
    boundary, and `per_family` matrices of every profile of the batch."""
    batch = len(labels)
    idx = {0, batch - 1, min(7, batch - 1), min(8, batch - 1), max(batch - 9, 0), max(batch - 8, 0)}
    for fam in sorted(set(labels)):
        members = [i for i, lab in enumerate(labels) if lab == fam]
        k = min(per_family, len(members))
        idx.update(members[(j * (len(members) - 1)) // max(k - 1, 1)] for j in range(k))
    return sorted(idx)


# The task's 12 benchmark cases (official/task.yml:109-121): the whole batch
# through custom_kernel (the schedule bench.py times), the oracle on every
# matrix for n <= 352 and on a stratified sample above (every profile of the
# mixed batches, batch boundaries).
@pytest.mark.parametrize("case", cases.BENCHMARKS, ids=[c.label for c in cases.BENCHMARKS])
def test_official_benchmark_case(cuda, case):
    a = cases.generate(case)
    labels = cases.labels_of(case)
    sample = list(range(case.batch)) if case.n <= 352 else stratified_sample(labels)
    print(f"[official benchmark] {case.label}: full batch, checking {len(sample)} matrices", flush=True)
    d = a.to(cuda)
    h, tau = custom_kernel(d)
    torch.cuda.synchronize()
    sel = torch.tensor(sample)
    a, h, tau = a[sel], h[sel.to(cuda)].cpu(), tau[sel.to(cuda)].cpu()
    del d
    ok, msg = checker.official_check(a, h, tau)
    assert ok, msg
    h_ref, tau_ref = torch.geqrf(a)
    ag = checker.rdiag_tau_agreement(a, h, tau, h_ref, tau_ref)
    assert ag.ok, ag.message()


# The explicit Q on every profile: fastqr.householder_product of the GPU
# factors against the oracle (CPU torch.linalg.householder_product in fp64 of
# the same factors), ||Q - Q_ref||_F <= 1e-5 n.
@pytest.mark.parametrize("case", cases.TESTS, ids=[c.label for c in cases.TESTS])
def test_official_case_explicit_q(cuda, case):
    import fastqr

    print(f"[official Q] {case.label}", flush=True)
    a = cases.generate(case)
    h, tau = custom_kernel(a.to(cuda))
    q = fastqr.householder_product(h, tau)
    torch.cuda.synchronize()
    q_ref = torch.linalg.householder_product(h.cpu().double(), tau.cpu().double())
    err = torch.linalg.matrix_norm(q.cpu().double() - q_ref).max().item()
    assert err <= 1e-5 * case.n, f"||Q - Q_ref||_F = {err:.3e}"


# The evaluator's benchmark loop (fastqr.evaluator, official/eval.py:157-251)
# on two of the task's benchmark cases with a short time budget: the warm-up
# case, the pre-timing check, flushed and event-timed repeats, the bitwise
# recheck of every timed output, the stopping rule.
def test_evaluator_loop_on_two_cases(cuda):
    from fastqr import evaluator

    print("[evaluator] 20x32 and 40x176", flush=True)
    specs = [cases.BENCHMARKS[0], cases.BENCHMARKS[1]]
    dev = evaluator.torch_device(torch, custom_kernel, checker.official_check, flush_bytes=1 << 28)
    results, passed = evaluator.run_benchmarking(specs, lambda c: cases.generate(c).to(cuda), dev,
                                                 recheck="bitwise", check_matrices=4, max_repeats=50,
                                                 max_time_ns=2e7, warmup_max_time_ns=1e7)
    assert passed, results
    for spec, st in zip(specs, results):
        assert isinstance(st, evaluator.Stats) and st.runs >= 3, st
        assert 0 < st.best <= st.mean <= st.worst
        print(f"  {spec.label}: mean {st.mean / 1e3:.1f} us over {st.runs} repeats", flush=True)
