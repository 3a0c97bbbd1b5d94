"""Seeded parameter initialization (synaptik_amd/initializers.py, csrc/lxm.cpp).

Pinned against the reference's own tests:
  * the initializer transforms through stub sources, as LinearInitializationTest.java:40-153 and
    ParameterInitializersTest.java:113-197 assert them: the bound or deviation each draw is asked
    for (fanOut = dim 0, fanIn = dim 1, binary64 arithmetic), the number and order of draws, the
    single narrowing of mean + g * deviation, validation that consumes no draw, a failing source;
  * the builder's step seeds (ModelBuilderTest.java:63-91): the Linear at step 2 of
    linear(3).relu().linear(3) with seed 7 is glorotUniform([3, 3]) from a generator created with
    7 + 0x9E3779B97F4A7C15 * 2, biases are zero, seed 0 is the default.
The L64X128MixRandom stream itself has no literal draws in the reference and no JVM exists here:
it is "parity unpinned". Its parts are checked against what is published or fixed by the
mathematics: the SplitMix64 output sequence (Stafford's mixer), the LCG's closed-form jump, the
xoroshiro step's GF(2) linearity, the 53-bit grid of nextDouble and the half-open range of
nextDouble(origin, bound), and uniformity."""
import math

import numpy as np
import pytest
from scipy import stats

from synaptik_amd import initializers as I
from synaptik_amd.training import Dense, MlpSpec

GOLDEN = 0x9E3779B97F4A7C15
M64 = (1 << 64) - 1


class BoundedSource:
    """RandomGenerator stub: nextDouble(origin, bound) records its arguments and returns
    `value` (or values[i]); any other draw is an error; optionally fails on one call."""

    def __init__(self, calls=None, value=0.0, values=None, throw_on=None):
        self.values, self.value, self.throw_on = values, value, throw_on
        self.origins, self.bounds = [], []

    def calls(self):
        return len(self.origins)

    def next_double(self, origin=None, bound=None):
        assert origin is not None, "unbounded nextDouble must not be called"
        call = len(self.origins)
        self.origins.append(origin)
        self.bounds.append(bound)
        if call == self.throw_on:
            raise DeliberateSourceFailure()
        return self.values[call] if self.values is not None else self.value

    def next_gaussian(self):
        raise AssertionError("nextGaussian must not be called")

    def assert_calls(self, origin, bound, count):
        assert self.calls() == count
        assert all(o == origin for o in self.origins) and all(b == bound for b in self.bounds)


class GaussianSource:
    def __init__(self, *values, throw_on=None):
        self.values, self.n, self.throw_on = values, 0, throw_on

    def next_gaussian(self):
        call = self.n
        self.n += 1
        if call == self.throw_on:
            raise DeliberateSourceFailure()
        return self.values[call]

    def next_double(self, *a):
        raise AssertionError("nextDouble must not be called")


class DeliberateSourceFailure(RuntimeError):
    pass


# ---- initializer transforms (reference stub-source assertions) ----
@pytest.mark.parametrize("dt", ["FLOAT64", "FLOAT32"])
def test_linear_glorot_uniform_draws_six_calls_with_the_glorot_bound(dt):
    # LinearInitializationTest.java:40-76: Linear(in 2, out 3) -> weight [3, 2], 6 draws on
    # [-sqrt(6 / (2 + 3)), +sqrt(6 / (2 + 3))), zero bias
    src = BoundedSource(value=0.0)
    spec = MlpSpec([Dense(2, 3, None, bias=True)])
    w = I.glorot_uniform((3, 2), dt, src)
    b = I.zeros((3,), dt)
    bound = math.sqrt(6.0 / (2.0 + 3.0))
    src.assert_calls(-bound, bound, 6)
    assert w.shape == (3, 2) and b.shape == (3,) and spec.layers[0].fan_out == 3
    assert not w.any() and not b.any()
    assert w.dtype == {"FLOAT64": np.float64, "FLOAT32": np.float32}[dt]


def test_no_bias_linear_consumes_only_weight_draws():
    # LinearInitializationTest.java:78-95: Linear(in 4, out 2, no bias) -> 8 draws
    src = BoundedSource()
    I.glorot_uniform((2, 4), "FLOAT32", src)
    assert src.calls() == 8


def test_validation_fails_before_any_draw():
    # LinearInitializationTest.java:97-126, :128-138 and ParameterInitializers.java:375-402
    src = BoundedSource()
    with pytest.raises(TypeError, match="randomGenerator"):
        I.glorot_uniform((3, 2), "FLOAT32", None)
    for shape in ((0, 2), (3, 0)):
        with pytest.raises(ValueError, match="outFeatures" if shape[0] == 0 else "inFeatures"):
            I.glorot_uniform(shape, "FLOAT32", src)
    with pytest.raises(ValueError, match="floating"):
        I.glorot_uniform((1, 1), "INT32", src)
    with pytest.raises(ValueError, match="rank-two"):
        I.glorot_uniform((2, 2, 2), "FLOAT32", src)
    with pytest.raises(ValueError, match="Java array limit"):
        I.glorot_uniform((46_341, 46_341), "FLOAT64", src)
    assert src.calls() == 0


def test_failing_source_keeps_completed_draws_and_returns_nothing():
    # LinearInitializationTest.java:140-153: failure on call 2 -> 3 calls made, no tensor
    src = BoundedSource(throw_on=2)
    with pytest.raises(DeliberateSourceFailure):
        I.glorot_uniform((3, 2), "FLOAT64", src)
    assert src.calls() == 3


def test_normal_and_uniform_delegate_with_exact_arguments_and_one_narrowing():
    # ParameterInitializersTest.java:113-144
    gaussian = GaussianSource(-1.25, 0.5)
    uniform = BoundedSource(values=[-0.75, 0.25])
    mean = float.fromhex("0x1.0000000000001p4")
    deviation = float.fromhex("0x1.0000000000001p-4")
    got = I.normal((2,), "FLOAT32", mean, deviation, gaussian)
    want = np.array([mean + -1.25 * deviation, mean + 0.5 * deviation]).astype(np.float32)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    assert gaussian.n == 2
    bounded = I.uniform((2,), "FLOAT32", -2.25, 3.75, uniform)
    uniform.assert_calls(-2.25, 3.75, 2)
    assert bounded.tolist() == [-0.75, 0.25]


def test_initialize_dispatches_policies():
    # ParameterInitializersTest.java:146-197
    gaussian = GaussianSource(-1.0, 2.0)
    uniform = BoundedSource(values=[-0.5, 0.75])
    P = I.ParameterInitialization
    assert I.initialize((2,), "FLOAT32", P("zeros")).tolist() == [0.0, 0.0]
    assert I.initialize((2,), "FLOAT32", P("ones")).tolist() == [1.0, 1.0]
    assert I.initialize((2,), "FLOAT64", P("normal", 2.0, 0.5), gaussian).tolist() == [1.5, 3.0]
    assert I.initialize((2,), "FLOAT64", P("uniform", -2.0, 3.0), uniform).tolist() == [-0.5, 0.75]
    assert gaussian.n == 2
    uniform.assert_calls(-2.0, 3.0, 2)
    with pytest.raises(ValueError):
        I.initialize((2,), "FLOAT32", P("glorot_uniform"))
    with pytest.raises(ValueError):
        I.initialize((2,), "FLOAT32", P("zeros"), gaussian)
    for args, name in ((((None, None, None)), "shape"), (((2,), None, None), "dataType"),
                       (((2,), "FLOAT32", None), "initialization")):
        with pytest.raises(TypeError, match=name):
            I.initialize(*args)


def test_fan_convention_bounds_and_row_major_draw_order():
    """fanOut = dim 0, fanIn = dim 1 (ParameterInitializers.java:269-372), values land in
    row-major order of [fanOut, fanIn]."""
    class Counting(BoundedSource):
        def next_double(self, origin=None, bound=None):
            super().next_double(origin, bound)
            return float(self.calls() - 1)

    class CountingGaussian:
        n = 0

        def next_gaussian(self):
            self.n += 1
            return float(self.n - 1)

    for fn, bound in ((I.glorot_uniform, math.sqrt(6.0 / (5.0 + 3.0))),
                      (I.kaiming_relu_uniform, math.sqrt(6.0 / 5.0))):
        src = Counting()
        w = fn((3, 5), "FLOAT64", src)
        src.assert_calls(-bound, bound, 15)
        assert np.array_equal(w, np.arange(15.0).reshape(3, 5))
    for fn, std in ((I.glorot_normal, math.sqrt(2.0 / (5.0 + 3.0))),
                    (I.kaiming_relu_normal, math.sqrt(2.0 / 5.0))):
        w = fn((3, 5), "FLOAT64", CountingGaussian())
        assert np.array_equal(w, (0.0 + np.arange(15.0) * std).reshape(3, 5))


def test_normal_and_uniform_argument_validation():
    src = BoundedSource()
    for lo, hi in ((math.nan, 1.0), (0.0, math.inf), (1.0, 1.0), (2.0, 1.0)):
        with pytest.raises(ValueError):
            I.uniform((2,), "FLOAT32", lo, hi, src)
    for mean, std in ((math.inf, 1.0), (0.0, -1.0), (0.0, math.nan)):
        with pytest.raises(ValueError):
            I.normal((2,), "FLOAT32", mean, std, GaussianSource(0.0, 0.0))
    assert src.calls() == 0


# ---- the builder's per-step generators ----
def test_builder_step_seeds_and_layer_generators():
    # ModelBuilderTest.java:63-91: linear(3).relu().linear(3) on input width 3, seed 7
    spec = MlpSpec([Dense(3, 3, "relu"), Dense(3, 3, None)])
    Ws, bs = I.builder_parameters(spec, 7)
    want = I.glorot_uniform((3, 3), "FLOAT32", I.L64X128MixRandom(7 + GOLDEN * 2 - (1 << 64)))
    assert np.array_equal(Ws[1].view(np.uint32), want.view(np.uint32))
    assert not Ws[0].tobytes() == Ws[1].tobytes()
    assert all(not b.any() for b in bs)
    again, _ = I.builder_parameters(spec, 7)  # builds are deterministic
    assert all(a.tobytes() == b.tobytes() for a, b in zip(Ws, again))
    zero, _ = I.builder_parameters(MlpSpec([Dense(2, 2)]))
    explicit, _ = I.builder_parameters(MlpSpec([Dense(2, 2)]), 0)
    assert zero[0].tobytes() == explicit[0].tobytes()
    # long wraparound of the step seed and layers without activation steps
    wrapped = (-1 + 3 * GOLDEN) & M64
    assert I.builder_step_seed(-1, 3) == (wrapped - (1 << 64) if wrapped >= 1 << 63 else wrapped)
    spec2 = MlpSpec([Dense(4, 5, None), Dense(5, 2, None, bias=False)])
    W2, b2 = I.builder_parameters(spec2, 11)
    want2 = I.glorot_uniform((2, 5), "FLOAT32", I.L64X128MixRandom(I.builder_step_seed(11, 1)))
    assert W2[1].tobytes() == want2.tobytes() and b2[1] is None


# ---- the L64X128MixRandom restatement ----
def _splitmix64(seed, n):
    out, s = [], seed
    for _ in range(n):
        s = (s + GOLDEN) & M64
        z = s
        z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & M64
        z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & M64
        out.append(z ^ (z >> 31))
    return out


def test_stafford_mixer_gives_the_published_splitmix64_sequence():
    """x0 and x1 of a seed are Stafford-13 mixes of seed' and seed' + golden ratio, i.e. the
    first two SplitMix64 outputs from seed' - golden ratio. SplitMix64 from seed 0 is
    0xe220a8397b1dcdaf, 0x6e789e6aa1b965f4, 0x06c45d188009454f (Vigna's reference
    implementation), so the mixer must reproduce them."""
    assert _splitmix64(0, 3) == [0xE220A8397B1DCDAF, 0x6E789E6AA1B965F4, 0x06C45D188009454F]
    silver = 0x6A09E667F3BCC909
    for seed in (0, 1, -1, 42, 7 + 2 * GOLDEN):
        v = (seed ^ silver) & M64
        a, s, x0, x1 = I.L64X128MixRandom(seed).state
        assert [x0, x1] == _splitmix64((v - GOLDEN) & M64, 2)
        assert s == 1 and a & 1 == 1


def test_lcg_part_follows_its_closed_form_and_xbg_part_is_linear():
    """After k outputs the LCG state is M^k s + a (M^k - 1)/(M - 1) mod 2^64 (a geometric sum,
    computed here by exact integer arithmetic); the xoroshiro step is linear over GF(2)."""
    Mul = 0xD1342543DE82EF95
    g = I.L64X128MixRandom(123)
    a, s, _, _ = g.state
    g.next_longs(1000)
    geo = sum(pow(Mul, i, 1 << 64) for i in range(1000)) & M64
    assert g.state[1] == (pow(Mul, 1000, 1 << 64) * s + a * geo) & M64

    def step(x0, x1):
        rot = lambda v, k: ((v << k) | (v >> (64 - k))) & M64
        q1 = x1 ^ x0
        q0 = rot(x0, 24) ^ q1 ^ ((q1 << 16) & M64)
        return q0, rot(q1, 37)

    h = I.L64X128MixRandom(5)
    x = h.state[2:]
    h.next_longs(1)
    assert h.state[2:] == step(*x)  # the generator advances its xor part by exactly one step
    rng = np.random.default_rng(0)
    for _ in range(50):
        u = [int(v) for v in rng.integers(0, 2**63, 4)]
        l, r = step(u[0], u[1]), step(u[2], u[3])
        assert step(u[0] ^ u[2], u[1] ^ u[3]) == (l[0] ^ r[0], l[1] ^ r[1])


def test_doubles_grid_range_and_uniformity():
    g = I.L64X128MixRandom(99)
    d = g.next_doubles(200_000)
    assert d.min() >= 0.0 and d.max() < 1.0
    assert np.all(d * 2.0**53 == np.floor(d * 2.0**53))  # multiples of 2^-53
    assert stats.kstest(d, "uniform").pvalue > 1e-4
    assert abs(np.corrcoef(d[:-1], d[1:])[0, 1]) < 0.01
    h = I.L64X128MixRandom(99)
    longs = h.next_longs(1000).view(np.uint64)
    assert np.array_equal((longs >> np.uint64(11)).astype(np.float64) * 2.0**-53, d[:1000])
    u = I.L64X128MixRandom(3).uniform_block(-0.25, 0.5, 100_000, np.float64)
    assert u.min() >= -0.25 and u.max() < 0.5
    assert stats.kstest((u + 0.25) / 0.75, "uniform").pvalue > 1e-4
    # nextDouble(origin, bound) = nextDouble() * (bound - origin) + origin, two roundings
    r = I.L64X128MixRandom(3).next_doubles(1000)
    assert np.array_equal(u[:1000], r * 0.75 + -0.25)
    # the binary32 narrowing is once, of the same draws
    f = I.L64X128MixRandom(3).uniform_block(-0.25, 0.5, 1000, np.float32)
    assert np.array_equal(f, u[:1000].astype(np.float32))
    with pytest.raises(ValueError):
        I.L64X128MixRandom(3).uniform_block(1.0, 1.0, 1, np.float64)
    with pytest.raises(ValueError):
        I.L64X128MixRandom(3).uniform_block(-1e308, 1e308, 1, np.float64)


def test_nearby_seeds_give_unrelated_streams():
    a = I.L64X128MixRandom(0).next_doubles(50_000)
    b = I.L64X128MixRandom(1).next_doubles(50_000)
    assert abs(np.corrcoef(a, b)[0, 1]) < 0.02
    ga = I.L64X128MixRandom(0).gaussian_block(50_000)
    gb = I.L64X128MixRandom(1).gaussian_block(50_000)
    assert abs(np.corrcoef(ga, gb)[0, 1]) < 0.02


# ---- nextGaussian: McFarland's modified ziggurat (tables from its construction) ----
def _f(x):
    return np.exp(-0.5 * np.asarray(x, np.float64) ** 2)


def test_ziggurat_layers_have_equal_area_and_fill_the_half_normal():
    """256 boxes of area A = sqrt(pi/2)/256: rectangle 0 is [0, x0] x [0, f(x0)], rectangle k is
    [0, x_k] x [f(x_{k-1}), f(x_k)], each of area A, widths strictly decreasing; no further
    rectangle of area A fits under the curve above the last; the tail, overhang and cap areas,
    integrated independently, add up with the rectangles to the whole half-normal area."""
    from scipy import integrate, special
    t = I.gaussian_tables()
    R, A, x = t["layers"], t["box_area"], t["x"]
    T = math.sqrt(math.pi / 2)
    assert A == pytest.approx(T / 256, rel=1e-15)
    assert R == 253 and x[R] == 0.0 and len(x) == R + 1
    assert np.all(np.diff(x) < 0)
    assert x[0] * _f(x[0]) == pytest.approx(A, rel=1e-13)
    assert x[0] > 1.0  # the larger root of x f(x) = A
    for k in range(1, R):
        assert x[k] * (_f(x[k]) - _f(x[k - 1])) == pytest.approx(A, rel=1e-9), k
    xs = np.linspace(0, x[R - 1], 200_001)
    assert np.max(xs * (_f(xs) - _f(x[R - 1]))) < A  # the cap holds no further rectangle
    area = t["region_area"]
    assert area[0] == pytest.approx(T * special.erfc(x[0] / math.sqrt(2)), rel=1e-9)
    for k in range(1, R):
        want = integrate.quad(lambda u: math.exp(-0.5 * u * u) - _f(x[k - 1]), x[k], x[k - 1],
                              epsabs=0, epsrel=1e-12)[0]
        assert area[k] == pytest.approx(want, rel=1e-7, abs=1e-16), k
    cap = integrate.quad(lambda u: math.exp(-0.5 * u * u) - _f(x[R - 1]), 0, x[R - 1],
                         epsabs=0, epsrel=1e-12)[0]
    assert area[R] == pytest.approx(cap, rel=1e-9)
    assert np.all(area > 0)
    assert R * A + area.sum() == pytest.approx(T, rel=1e-12)
    assert area.sum() == pytest.approx((256 - R) * A, rel=1e-9)


def test_ziggurat_alias_table_reproduces_the_region_probabilities():
    """Walker's alias table over 256 columns: each region's probability (column j kept with
    threshold_j / 2^56, else sent to alias_j) equals its area over the slow path's total."""
    t = I.gaussian_tables()
    R, thr, alias, area = t["layers"], t["threshold"], t["alias"], t["region_area"]
    keep = thr.astype(np.float64) / 2.0**56
    assert np.all((keep >= 0) & (keep <= 1)) and np.all(alias <= R)
    prob = np.zeros(R + 1)
    for j in range(256):
        if j <= R:
            prob[j] += keep[j] / 256
        else:
            assert keep[j] == 0.0  # unused columns always take their alias
        prob[alias[j]] += (1 - keep[j]) / 256
    np.testing.assert_allclose(prob, area / area.sum(), rtol=0, atol=2.0**-52)


def test_gaussian_fast_path_is_the_rectangle_closed_form():
    """A draw whose first nextLong picks a rectangle (low 8 bits < R) is x_box * U1 * 2^-63 of that
    one long and consumes nothing else; the slow path consumes at least two longs. Checked by
    following the long stream of an identically seeded generator."""
    t = I.gaussian_tables()
    R, x = t["layers"], t["x"]
    gen = I.L64X128MixRandom(1234)
    fast = slow = 0
    for _ in range(3000):
        c = I.L64X128MixRandom(0)
        c._state[:] = gen._state[:]
        v = gen.next_gaussian()
        u1 = c.next_long()
        box = u1 & 0xFF
        if box < R:
            assert v == math.ldexp(x[box], -63) * float(u1)
            assert gen.state == c.state  # exactly one long
            fast += 1
        else:
            assert math.copysign(1.0, v) == (-1.0 if u1 < 0 else 1.0)  # the sign is U1's
            assert gen.state != c.state  # more than the one long
            slow += 1
    assert fast + slow == 3000 and slow > 0
    assert fast / 3000 == pytest.approx(R / 256, abs=0.02)


def test_gaussian_draws_follow_the_standard_normal():
    """4M draws: moments, Kolmogorov-Smirnov against Phi, a chi-square over the ziggurat's own
    layer boundaries (which would see a wrong overhang or cap), the tail beyond x0 (its mass and,
    conditionally, its shape), and sign symmetry."""
    from scipy import special, stats
    t = I.gaussian_tables()
    x = t["x"]
    d = I.L64X128MixRandom(20240607).gaussian_block(4_000_000)
    n = d.size
    assert abs(d.mean()) < 5 / math.sqrt(n)
    assert d.var() == pytest.approx(1.0, abs=5 * math.sqrt(2 / n))
    assert abs(stats.skew(d)) < 5 * math.sqrt(6 / n)
    assert abs(stats.kurtosis(d)) < 5 * math.sqrt(24 / n)
    assert stats.kstest(d, "norm").pvalue > 1e-4
    a = np.abs(d)
    edges = np.concatenate([[0.0], x[::-1][1:], [np.inf]])  # 0 < x_{R-1} < ... < x_0 < inf
    counts = np.histogram(a, edges)[0]
    cdf = special.erf(edges / math.sqrt(2))
    expect = n * np.diff(cdf)
    assert stats.chisquare(counts, expect).pvalue > 1e-4
    tail = a[a > x[0]]
    assert tail.size == pytest.approx(n * special.erfc(x[0] / math.sqrt(2)), rel=0.15)
    # conditional tail: P(|g| > s | |g| > x0) = erfc(s/sqrt2) / erfc(x0/sqrt2)
    assert stats.kstest(tail, lambda s: 1 - special.erfc(s / math.sqrt(2)) /
                        special.erfc(x[0] / math.sqrt(2))).pvalue > 1e-4
    assert abs((d > 0).mean() - 0.5) < 5 * 0.5 / math.sqrt(n)


def test_normal_policies_draw_from_the_generator_in_row_major_order():
    """kaimingReluNormal / glorotNormal / normal over L64X128MixRandom: one nextGaussian per
    element in row-major order, (type)(mean + g * deviation) narrowed once
    (TensorRandoms.java:615-656); the next draw after the tensor is the generator's next one."""
    seed = I.builder_step_seed(7, 2)
    src = I.L64X128MixRandom(seed)
    w = I.kaiming_relu_normal((3, 5), "FLOAT32", src)
    ref = I.L64X128MixRandom(seed).gaussian_block(16)
    std = math.sqrt(2.0 / 5.0)
    assert np.array_equal(w, (0.0 + ref[:15] * std).astype(np.float32).reshape(3, 5))
    assert src.next_gaussian() == ref[15]
    g = I.glorot_normal((4, 2), "FLOAT64", I.L64X128MixRandom(11))
    ref = I.L64X128MixRandom(11).gaussian_block(8)
    assert np.array_equal(g, (ref * math.sqrt(2.0 / 6.0)).reshape(4, 2))
    v = I.initialize((6,), "FLOAT32", I.ParameterInitialization("normal", 1.5, 0.25),
                     I.L64X128MixRandom(3))
    assert np.array_equal(v, (1.5 + I.L64X128MixRandom(3).gaussian_block(6) * 0.25).astype(np.float32))
    # a per-element source gives the same tensor as the block draw
    class PerElement:
        def __init__(self, seed):
            self.g = I.L64X128MixRandom(seed)

        def next_gaussian(self):
            return self.g.next_gaussian()

    assert np.array_equal(I.kaiming_relu_normal((3, 5), "FLOAT32", PerElement(seed)), w)


def test_builder_he_normal_parameters_use_the_step_seeds():
    from synaptik_amd.training import MlpSpec, init_parameters
    spec = MlpSpec.chain([6, 4, 3], hidden="relu", loss="ce")
    Ws, bs = init_parameters(spec, 5, "builder_he_normal")
    # steps: linear 0, relu 1, linear 2
    for W, step, fan_in in ((Ws[0], 0, 6), (Ws[1], 2, 4)):
        ref = I.L64X128MixRandom(I.builder_step_seed(5, step)).gaussian_block(W.size)
        assert np.array_equal(W, (ref * math.sqrt(2.0 / fan_in)).astype(np.float32).reshape(W.shape))
    assert all(b is not None and not b.any() for b in bs)
