"""Random programs through the schedule check: seeded step sequences over a small pool of slots,
so that later steps overwrite what earlier ones read or write (every read-after-write,
write-after-read and write-after-write pattern across the two streams), mixed with large GEMMs
that stay on the context stream, optimizer passes that OR into or read the status word, loss
MEANs and trailing commits the run's last launch performs. For each, the plan program creation
makes (shk_hip_program_plan, no device) must order every conflicting pair of steps
(tests/plan_hazards.py). The runtime's own dependency model is coarser than the check's -- it
orders two status readers, and treats every tensor of an optimizer entry as read and written --
so on such programs some of its waits are conservative; on the lowered programs of
test_plan_hazards_cpu.py every wait is needed."""
import numpy as np
import pytest

from synaptik_amd.native import HipBackendError, program_plan, validate_program_image
from synaptik_amd.program import ProgramBuilder
from tests import plan_hazards as H
from tests.conftest import needs_two_streams

SMALL = 64 * 64      # floats of a small slot: a 64 x 64 matrix
BIG = 1024 * 1024    # floats of a big slot: a 1024 x 1024 matrix (GEMMs of 2^30 multiply-adds)


def _program(seed: int) -> bytes:
    rng = np.random.default_rng(seed)
    pb = ProgramBuilder()
    small_ro = [pb.input(SMALL) for _ in range(2)]
    small_rw = [pb.input(SMALL, inout=True) for _ in range(2)] + \
        [pb.internal(SMALL) for _ in range(int(rng.integers(4, 7)))] + [pb.output(SMALL)]
    big_rw = [pb.internal(BIG) for _ in range(3)]
    big_ro = [pb.input(BIG)]
    counter = pb.input(1, "i64", inout=True)
    loss = pb.output(1)

    def pick(pool, exclude=()):
        choices = [s for s in pool if s not in exclude]
        return choices[int(rng.integers(len(choices)))]

    for _ in range(int(rng.integers(6, 22))):
        op = int(rng.integers(0, 10))
        if op == 0:
            src = pick(small_ro + small_rw)
            pb.copy(src, pick(small_rw, (src,)), SMALL)
        elif op == 1:
            pb.fill(pick(small_rw), SMALL, float(rng.integers(0, 3)))
        elif op == 2:
            src = pick(small_ro + small_rw)
            pb.reduce_all(src, pick(small_rw, (src,)), SMALL, "sum")
        elif op == 3:
            src = pick(small_ro + small_rw)
            pb.colsum(src, pick(small_rw, (src,)), 64, 64, accumulate=bool(rng.integers(2)))
        elif op == 4:  # a small GEMM, side-stream material
            a, b = pick(small_ro + small_rw), pick(small_ro + small_rw)
            pb.gemm(a, b, pick(small_rw, (a, b)), 64, 64, 64, trans_b=bool(rng.integers(2)))
        elif op == 5:  # a large GEMM: stays on the context stream
            a, b = pick(big_ro + big_rw), pick(big_ro + big_rw)
            pb.gemm(a, b, pick(big_rw, (a, b)), 1024, 1024, 1024)
        elif op == 6:  # a staged optimizer pass (ORs into the status word)
            p_, g = pick(small_rw), pick(small_ro + small_rw)
            pn = pick(small_rw, (p_, g))
            kind = ["sgd", "adam"][int(rng.integers(2))]
            m = pick(small_rw, (p_, g, pn))
            mn = pick(small_rw, (p_, g, pn, m))
            if kind == "adam":
                v = pick(small_rw, (p_, g, pn, m, mn))
                vn = pick(small_rw, (p_, g, pn, m, mn, v))
            else:
                v = vn = None
            pb.optimizer(counter, [(p_, g, m, v, pn, mn, vn, SMALL)], kind=kind, phase=2,
                         lr=0.01, momentum=0.9 if kind == "sgd" else 0.0,
                         has_momentum_slot=kind == "sgd")
        elif op == 7:  # accumulator commit / clear (read the status word), or accumulate (OR)
            g, m = pick(small_ro + small_rw), pick(small_rw)
            while m is g:
                m = pick(small_rw)
            kind = ["acc_sum", "acc_commit", "acc_clear"][int(rng.integers(3))]
            if kind == "acc_sum":
                pb.optimizer(counter, [(pick(small_rw, (g, m)), g, m, None, SMALL)], kind=kind,
                             phase=0, lr=0.0)
            else:  # the kernel leaves the parameter alone, the image still names one
                pb.optimizer(counter, [(pick(small_rw, (g, m)), g, m, None, SMALL)], kind=kind,
                             phase=0, lr=0.0)
        elif op == 8:  # an MSE (loss + gradient)
            p_, t = pick(small_ro + small_rw), pick(small_ro + small_rw)
            pb.mse(p_, t, loss, SMALL, grad=pick(small_rw, (p_, t)))
        else:  # the CE head's loss MEAN over per-row losses
            pb.ce_head_loss(pick(small_ro + small_rw), loss, 64)
    if rng.random() < 0.6:
        pb.step_commit(counter)
    return pb.image()


def _cases(n):
    out = []
    for seed in range(n):
        img = _program(seed)
        try:
            validate_program_image(img)
        except HipBackendError:
            continue  # a combination the image validator refuses (not a schedule question)
        out.append((seed, img))
    return out


@pytest.fixture(scope="module")
def cases():
    return _cases(400)


def test_generator_yields_valid_two_stream_programs(cases):
    assert len(cases) >= 300
    side = sum(1 for _, img in cases if any(program_plan(img)[0]))
    assert side >= len(cases) // 2


@needs_two_streams
def test_random_programs_are_race_free(cases):
    for seed, img in cases:
        steps = H.decode(img)
        stream_of, wait_for, folded = program_plan(img)
        hazards = H.check_plan(steps, stream_of, wait_for, folded)
        assert not hazards, (seed, [str(h) for h in hazards[:3]])
