"""Seeded random MATMUL partitions through the SPI mirror on the GPU: the forward pattern
X.PERMUTE(W) (+ bias) (+ activation), the weight-gradient pattern PERMUTE(PERMUTE(X).G), the
input-gradient pattern G.PERMUTE(PERMUTE(W)), two-layer chains, published intermediates (which
stop a fusion), and stand-alone PERMUTEs, with ragged extents. Integer-valued operands make every
GEMM exact, so each output must equal the numpy evaluation of the same graph bit for bit; an output
downstream of TANH or SIGMOID (binary64-evaluated and narrowed once, by two binary64 libraries)
within 2 ulp."""
import numpy as np
import pytest

from oracle import oracle
from synaptik_amd.backend import (HipPartitionFinalizer, HipPartitionPreparer, Node, Partition,
                                  TensorDescriptor as T)

pytestmark = pytest.mark.gpu

DIMS = [1, 2, 5, 16, 17, 64, 100, 128, 257]
ACTS = {"RELU": "relu", "TANH": "tanh", "SIGMOID": "sigmoid"}


def f32(*s):
    return T("FLOAT32", tuple(s))


def _ints(rng, *shape):
    return rng.integers(-3, 4, size=shape).astype(np.float32)


def _graph(seed):
    rng = np.random.default_rng(900 + seed)
    M, K, N, N2 = (int(rng.choice(DIMS)) for _ in range(4))
    vals, nodes, feed, env, outs = {}, [], {}, {}, []

    def inp(name, arr):
        vals[name] = f32(*arr.shape)
        feed[name] = arr
        env[name] = arr

    def node(kind, ins, out, shape, value, attrs=None):
        vals[out] = f32(*shape)
        nodes.append(Node(kind, ins, out, attrs or {}))
        env[out] = value.astype(np.float32)

    pattern = int(rng.integers(0, 4))
    if pattern == 0:  # forward layer
        inp("X", _ints(rng, M, K)); inp("W", _ints(rng, N, K))
        node("PERMUTE", ["W"], "WT", (K, N), env["W"].T, {"axes": (1, 0)})
        node("MATMUL", ["X", "WT"], "Z", (M, N), oracle.matmul(env["X"], env["W"], trans_b=True))
        last = "Z"
        if rng.random() < 0.7:
            inp("b", (rng.integers(-4, 5, N) * 0.25).astype(np.float32))
            node("ADD", [last, "b"], "Zb", (M, N), env[last] + env["b"][None, :])
            last = "Zb"
            if rng.random() < 0.3:
                outs.append("Zb")  # published: the activation cannot fuse into the GEMM
        if rng.random() < 0.7:
            a = str(rng.choice(list(ACTS)))
            node(a, [last], "Y", (M, N), oracle.activation(ACTS[a], env[last]))
            last = "Y"
        outs.append(last)
    elif pattern == 1:  # weight gradient written as [N, K]
        inp("X", _ints(rng, M, K)); inp("G", _ints(rng, M, N))
        node("PERMUTE", ["X"], "XT", (K, M), env["X"].T, {"axes": (1, 0)})
        node("MATMUL", ["XT", "G"], "dWT", (K, N), oracle.matmul(env["X"], env["G"], trans_a=True))
        node("PERMUTE", ["dWT"], "dW", (N, K), env["dWT"].T, {"axes": (1, 0)})
        outs.append("dW")
        if rng.random() < 0.3:
            outs.append("dWT")  # both the product and its permutation published
    elif pattern == 2:  # input gradient G . (W^T)^T
        inp("G", _ints(rng, M, N)); inp("W", _ints(rng, N, K))
        node("PERMUTE", ["W"], "WT", (K, N), env["W"].T, {"axes": (1, 0)})
        node("PERMUTE", ["WT"], "WTT", (N, K), env["W"], {"axes": (1, 0)})
        node("MATMUL", ["G", "WTT"], "dX", (M, K), oracle.matmul(env["G"], env["W"]))
        outs.append("dX")
        if rng.random() < 0.3:
            outs.append("WT")  # a permutation that is also published: materialized
    else:  # two layers
        inp("X", _ints(rng, M, K)); inp("W1", _ints(rng, N, K)); inp("W2", _ints(rng, N2, N))
        inp("b1", (rng.integers(-4, 5, N) * 0.5).astype(np.float32))
        node("PERMUTE", ["W1"], "W1T", (K, N), env["W1"].T, {"axes": (1, 0)})
        node("MATMUL", ["X", "W1T"], "Z1", (M, N), oracle.matmul(env["X"], env["W1"], trans_b=True))
        node("ADD", ["Z1", "b1"], "Z1b", (M, N), env["Z1"] + env["b1"][None, :])
        node("RELU", ["Z1b"], "Y1", (M, N), oracle.activation("relu", env["Z1b"]))
        node("PERMUTE", ["W2"], "W2T", (N, N2), env["W2"].T, {"axes": (1, 0)})
        node("MATMUL", ["Y1", "W2T"], "Z2", (M, N2), oracle.matmul(env["Y1"], env["W2"], trans_b=True))
        outs.append("Z2")
        if rng.random() < 0.4:
            outs.append("Y1")
    inputs = [v for v in feed]
    outs = list(dict.fromkeys(outs))
    return Partition(vals, nodes, inputs, outs), feed, env


@pytest.mark.parametrize("seed", range(64))
def test_random_matmul_partition(ctx, seed):
    part, feed, env = _graph(seed)
    print(f"matmul partition seed={seed} nodes={[n.kind for n in part.nodes]} "
          f"shapes={[tuple(part.values[v].shape) for v in part.inputs]} outputs={part.outputs}", flush=True)
    exe = HipPartitionFinalizer(ctx).finalize_partition(HipPartitionPreparer().analyze(part))
    got = exe.run_values(feed)
    transcendental = any(n.kind in ("TANH", "SIGMOID") for n in part.nodes)
    for v in part.outputs:
        g = np.ascontiguousarray(np.asarray(got[v], np.float32).reshape(env[v].shape))
        e = np.ascontiguousarray(env[v])
        if transcendental:
            ulps = np.abs(g.view(np.int32).astype(np.int64) - e.view(np.int32).astype(np.int64))
            assert ulps.max(initial=0) <= 2, (v, int(ulps.max()))
        else:
            assert np.array_equal(g.view(np.uint32), e.view(np.uint32)), v
    exe.close()
