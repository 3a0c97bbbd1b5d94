"""Seeded random elementwise partitions through the SPI mirror (preparer -> finalizer -> prepared
executable) on the GPU: DAGs of unary, binary, comparison and WHERE nodes over [R, C] values with
row, column and scalar broadcast operands and constants, values used once or several times (so the
lowering forms fused groups of varying size and splits groups that exceed its limits), some
intermediate values published, and a row or whole-tensor reduction of the last value. Elementwise
results must match a numpy evaluation of the same graph with the reference's per-operation
semantics (binary32 rounding per operation, binary64-evaluated transcendentals narrowed once,
Java Math.max) to within 2 ulp (exp / log / tanh evaluated by two binary64 libraries), NaN where
it is NaN; reductions within 1e-6 relative."""
import numpy as np
import pytest

from oracle import oracle
from synaptik_amd.backend import (HipPartitionFinalizer, HipPartitionPreparer, Node, Partition,
                                  TensorDescriptor as T)

pytestmark = pytest.mark.gpu

UNARY = ["NEG", "RELU", "TANH", "SIGMOID", "EXP", "LOG", "SQRT"]
BINARY = ["ADD", "SUB", "MUL", "DIV", "MAXIMUM"]


def _java_max(a, b):
    both_zero = (a == 0) & (b == 0)
    anded = (a.view(np.uint32) & b.view(np.uint32)).view(np.float32)
    m = np.where(a > b, a, b)
    m = np.where(both_zero, anded, m)
    m = np.where(np.isnan(b), b, m)
    return np.where(np.isnan(a), a, m).astype(np.float32)


def _unary(op, a):
    with np.errstate(all="ignore"):
        if op == "NEG":
            return (-a).astype(np.float32)
        if op in ("RELU", "TANH", "SIGMOID"):
            return oracle.activation(op.lower(), a.astype(np.float32))
        f = {"EXP": np.exp, "LOG": np.log, "SQRT": np.sqrt}[op]
        return f(a.astype(np.float64)).astype(np.float32)


def _binary(op, a, b):
    with np.errstate(all="ignore"):
        if op == "MAXIMUM":
            a, b = np.broadcast_arrays(a, b)
            return _java_max(np.ascontiguousarray(a), np.ascontiguousarray(b))
        return {"ADD": np.add, "SUB": np.subtract, "MUL": np.multiply, "DIV": np.divide}[op](a, b).astype(np.float32)


def _graph(seed):
    rng = np.random.default_rng(500 + seed)
    R, C = int(rng.choice([1, 3, 17, 64, 257])), int(rng.choice([1, 4, 10, 33, 128, 1000]))
    vals = {"x0": T("FLOAT32", (R, C)), "x1": T("FLOAT32", (R, C)), "row": T("FLOAT32", (C,)),
            "col": T("FLOAT32", (R, 1))}
    feed = {"x0": rng.standard_normal((R, C)).astype(np.float32) * 2,
            "x1": rng.standard_normal((R, C)).astype(np.float32) * 2,
            "row": rng.standard_normal(C).astype(np.float32),
            "col": rng.standard_normal((R, 1)).astype(np.float32)}
    env = dict(feed)
    full = ["x0", "x1"]
    nodes = []
    n_nodes = int(rng.integers(3, 14))
    for i in range(n_nodes):
        name = f"v{i}"
        kind = rng.random()
        if kind < 0.35:
            op = str(rng.choice(UNARY))
            a = str(rng.choice(full))
            nodes.append(Node(op, [a], name))
            env[name] = _unary(op, env[a])
        elif kind < 0.8:
            op = str(rng.choice(BINARY))
            a = str(rng.choice(full))
            r = rng.random()
            if r < 0.15:
                b = "row"
            elif r < 0.3:
                b = "col"
            elif r < 0.4:
                b = f"k{i}"
                vals[b] = T("FLOAT32", ())
                cval = float(np.float32(rng.choice([0.5, 2.0, -1.5, 3.0])))
                nodes.append(Node("CONSTANT", [], b, {"value": cval}))
                env[b] = np.float32(cval)
            else:
                b = str(rng.choice(full))
            if rng.random() < 0.5:
                a, b = b, a
            # a broadcast operand may stand first only if the output keeps the full shape
            nodes.append(Node(op, [a, b], name))
            env[name] = _binary(op, env[a], env[b])
        else:
            a, b, c, d = (str(rng.choice(full)) for _ in range(4))
            m = f"m{i}"
            vals[m] = T("BOOL", (R, C))
            nodes.append(Node("GREATER_THAN", [a, b], m))
            nodes.append(Node("WHERE", [m, c, d], name))
            env[name] = np.where(env[a] > env[b], env[c], env[d]).astype(np.float32)
        vals[name] = T("FLOAT32", (R, C))
        full.append(name)
    last = f"v{n_nodes - 1}"
    outputs = [last]
    for v in full[2:-1]:
        if rng.random() < 0.25:
            outputs.append(v)
    red = str(rng.choice(["SUM", "MEAN", "MAX", "none"]))
    axes = None if rng.random() < 0.5 else (-1,)
    if red != "none":
        vals["red"] = T("FLOAT32", () if axes is None else (R,))
        nodes.append(Node(red, [last], "red", {"axes": axes} if axes else {}))
        outputs.append("red")
    return Partition(vals, nodes, ["x0", "x1", "row", "col"], outputs), feed, env, red, axes


@pytest.mark.parametrize("seed", range(128))
def test_random_elementwise_partition(ctx, seed):
    part, feed, env, red, axes = _graph(seed)
    print(f"partition seed={seed} nodes={[n.kind for n in part.nodes]} outputs={part.outputs}", flush=True)
    exe = HipPartitionFinalizer(ctx).finalize_partition(HipPartitionPreparer().analyze(part))
    got = exe.run_values(feed)
    for v in part.outputs:
        g = np.asarray(got[v], np.float32)
        if v == "red":
            x = env[part.nodes[-1].inputs[0]]
            with np.errstate(all="ignore"):
                if red == "MAX":
                    w = (np.max(x) if axes is None else np.max(x, axis=-1)).astype(np.float32)
                    w = np.where(np.isnan(x).any() if axes is None else np.isnan(x).any(axis=-1), np.nan, w)
                else:
                    f = np.sum if red == "SUM" else np.mean
                    w = (f(x.astype(np.float64)) if axes is None else f(x.astype(np.float64), axis=-1)).astype(np.float32)
            g, w = np.atleast_1d(g).ravel(), np.atleast_1d(np.asarray(w, np.float32)).ravel()
            assert np.array_equal(np.isnan(g), np.isnan(w)), v
            fin = np.isfinite(w) & np.isfinite(g)
            np.testing.assert_allclose(g[fin], w[fin], rtol=1e-6, atol=1e-6 * (np.abs(x[np.isfinite(x)]).sum() + 1e-30) / max(x.size, 1))
            assert np.array_equal(g[~np.isfinite(w) & ~np.isnan(w)], w[~np.isfinite(w) & ~np.isnan(w)])
            continue
        w = np.asarray(env[v], np.float32).reshape(g.shape)
        assert np.array_equal(np.isnan(g), np.isnan(w)), v
        ok = ~np.isnan(w)
        inf = np.isinf(w) & ok
        assert np.array_equal(g[inf], w[inf]), v
        fin = ok & ~inf
        np.testing.assert_array_max_ulp(g[fin], w[fin], maxulp=2)
    exe.close()
