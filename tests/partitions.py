"""Compiler-shaped partitions (node lists as the reference's autograd emits them) for SPI tests."""
from synaptik_amd.backend import Node, Partition, TensorDescriptor as T


def f32(*shape):
    return T("FLOAT32", tuple(shape))


def mlp_train_partition(B, I, H, O):
    """Two Linear layers (ReLU, identity), MSE MEAN, and the gradient graph the reference's rules
    build: LinearAlgebraGradientRules (dX = dZ.(W^T)^T, d(W^T) = X^T.dZ then PERMUTE),
    ElementwiseGradientRules (ADD -> SUM_TO_SHAPE; RELU -> WHERE(x > 0, g, 0)),
    LossGradientRules (MSE: (p - t) * 2 * (g / count))."""
    v = {"x": f32(B, I), "W1": f32(H, I), "b1": f32(H), "W2": f32(O, H), "b2": f32(O), "t": f32(B, O),
         "W1T": f32(I, H), "Z1": f32(B, H), "Z1b": f32(B, H), "Y1": f32(B, H),
         "W2T": f32(H, O), "Z2": f32(B, O), "P": f32(B, O), "L": f32(),
         "D": f32(B, O), "two": f32(), "D2": f32(B, O), "one": f32(), "cnt": f32(), "gn": f32(),
         "dP": f32(B, O), "Y1T": f32(H, B), "dW2T": f32(H, O), "dW2": f32(O, H), "db2": f32(O),
         "W2TT": f32(O, H), "dY1": f32(B, H), "zero": f32(), "mask": T("BOOL", (B, H)),
         "dZ1": f32(B, H), "xT": f32(I, B), "dW1T": f32(I, H), "dW1": f32(H, I), "db1": f32(H)}
    n = [
        Node("PERMUTE", ["W1"], "W1T", {"axes": (1, 0)}),
        Node("MATMUL", ["x", "W1T"], "Z1"),
        Node("ADD", ["Z1", "b1"], "Z1b"),
        Node("RELU", ["Z1b"], "Y1"),
        Node("PERMUTE", ["W2"], "W2T", {"axes": (1, 0)}),
        Node("MATMUL", ["Y1", "W2T"], "Z2"),
        Node("ADD", ["Z2", "b2"], "P"),
        Node("MEAN_SQUARED_ERROR", ["P", "t"], "L", {"reduction": "MEAN"}),
        Node("SUB", ["P", "t"], "D"),
        Node("CONSTANT", [], "two", {"value": 2.0}),
        Node("MUL", ["D", "two"], "D2"),
        Node("CONSTANT", [], "one", {"value": 1.0}),
        Node("CONSTANT", [], "cnt", {"value": float(B * O)}),
        Node("DIV", ["one", "cnt"], "gn"),
        Node("MUL", ["D2", "gn"], "dP"),
        Node("PERMUTE", ["Y1"], "Y1T", {"axes": (1, 0)}),
        Node("MATMUL", ["Y1T", "dP"], "dW2T"),
        Node("PERMUTE", ["dW2T"], "dW2", {"axes": (1, 0)}),
        Node("SUM_TO_SHAPE", ["dP"], "db2"),
        Node("PERMUTE", ["W2T"], "W2TT", {"axes": (1, 0)}),
        Node("MATMUL", ["dP", "W2TT"], "dY1"),
        Node("CONSTANT", [], "zero", {"value": 0.0}),
        Node("GREATER_THAN", ["Z1b", "zero"], "mask"),
        Node("WHERE", ["mask", "dY1", "zero"], "dZ1"),
        Node("PERMUTE", ["x"], "xT", {"axes": (1, 0)}),
        Node("MATMUL", ["xT", "dZ1"], "dW1T"),
        Node("PERMUTE", ["dW1T"], "dW1", {"axes": (1, 0)}),
        Node("SUM_TO_SHAPE", ["dZ1"], "db1"),
    ]
    return Partition(v, n, ["x", "W1", "b1", "W2", "b2", "t"], ["L", "P", "dW1", "db1", "dW2", "db2", "Z1b"])


def softmax_ce_partition(R, C):
    """SOFTMAX, its gradient y*(g - SUM(g*y)), LOG_SUM_EXP + MEAN, and index CE."""
    v = {"x": f32(R, C), "g": f32(R, C), "labels": T("INT64", (R,)), "p": f32(R, C),
         "gy": f32(R, C), "s": f32(R, 1), "gs": f32(R, C), "dx": f32(R, C), "lse": f32(R),
         "m": f32(), "ce": f32(), "lsm": f32(R, C)}
    n = [
        Node("SOFTMAX", ["x"], "p", {"axis": -1}),
        Node("MUL", ["g", "p"], "gy"),
        Node("SUM", ["gy"], "s", {"axes": (1,), "keepdims": True}),
        Node("SUB", ["g", "s"], "gs"),
        Node("MUL", ["p", "gs"], "dx"),
        Node("LOG_SUM_EXP", ["x"], "lse", {"axis": -1}),
        Node("MEAN", ["lse"], "m", {"axes": None}),
        Node("INDEX_CATEGORICAL_CROSS_ENTROPY_WITH_LOGITS", ["x", "labels"], "ce", {"reduction": "MEAN"}),
        Node("LOG_SOFTMAX", ["x"], "lsm", {"axis": -1}),
    ]
    return Partition(v, n, ["x", "g", "labels"], ["p", "dx", "lse", "m", "ce", "lsm"])
