"""SPI mirror on the CPU: capability decisions and the lowered step sequence (no device work)."""
import pytest

from synaptik_amd.backend import (HipCapabilityProvider, HipPartitionPreparer, Node,
                                  OperationCapabilityQuery as Q, Partition, TensorDescriptor as T,
                                  UnsupportedPartition)
from synaptik_amd.program import (OP_COLSUM, OP_GEMM, OP_MSE, OP_POINTWISE, OP_TRANSPOSE,
                                  OP_SOFTMAX, OP_ROW_REDUCE, OP_REDUCE_ALL, OP_CE_INDEX)
from tests.partitions import f32, mlp_train_partition, softmax_ce_partition


def test_capability_admits_the_fp32_mlp_op_set():
    p = HipCapabilityProvider()
    assert p.backend_id() == "hip"
    assert p.supports(Q("MATMUL", (f32(4, 3), f32(3, 5)), (f32(4, 5),)))
    assert not p.supports(Q("MATMUL", (T("FLOAT64", (4, 3)), T("FLOAT64", (3, 5))), (T("FLOAT64", (4, 5)),)))
    assert not p.supports(Q("MATMUL", (f32(2, 4, 3), f32(3, 5)), (f32(2, 4, 5),)))
    assert p.supports(Q("ADD", (f32(4, 5), f32(5)), (f32(4, 5),)))
    assert not p.supports(Q("ADD", (f32(4, 5), f32(4)), (f32(4, 5),)))
    assert p.supports(Q("GREATER_THAN", (f32(4, 5), f32()), (T("BOOL", (4, 5)),)))
    assert p.supports(Q("SOFTMAX", (f32(8, 10),), (f32(8, 10),), (("axis", -1),)))
    assert not p.supports(Q("SOFTMAX", (f32(8, 10),), (f32(8, 10),), (("axis", 0),)))
    assert p.supports(Q("INDEX_CATEGORICAL_CROSS_ENTROPY_WITH_LOGITS", (f32(8, 10), T("INT64", (8,))), (f32(),)))
    assert not p.supports(Q("CONV2D", (f32(1, 3, 8, 8),), (f32(1, 3, 8, 8),)))
    assert not p.supports(Q("MAX", (f32(4, 5),), (f32(5),), (("axes", (0,)),)))
    assert p.supports(Q("PERMUTE", (f32(4, 5),), (f32(5, 4),), (("axes", (1, 0)),)))


def test_mlp_training_partition_lowers_to_fused_steps():
    a = HipPartitionPreparer().analyze(mlp_train_partition(16, 8, 12, 4))
    from synaptik_amd.program import ProgramBuilder  # noqa: F401
    import struct
    nsteps = struct.unpack_from("<IIII", a.plan, 0)[3]
    nslots = struct.unpack_from("<IIII", a.plan, 0)[2]
    off = 16 + 24 * nslots
    ops = []
    for _ in range(nsteps):
        op, plen = struct.unpack_from("<II", a.plan, off)
        ops.append(op)
        off += 200 + ((plen + 7) // 8) * 8
    # forward: 2 GEMMs (bias fused in both); loss; pointwise chains; 2 dW GEMMs written as
    # swapped GEMMs; one materialized W2^T (PERMUTE of a PERMUTE); dY1 GEMM; column sums
    assert ops.count(OP_GEMM) == 5
    assert ops.count(OP_TRANSPOSE) == 1
    assert ops.count(OP_COLSUM) == 2
    assert ops.count(OP_MSE) == 1
    assert ops.count(OP_POINTWISE) >= 2
    assert [r.kind for r in a.requirements][-1] == "Workspace"


def test_softmax_partition_lowering():
    a = HipPartitionPreparer().analyze(softmax_ce_partition(32, 10))
    import struct
    nslots, nsteps = struct.unpack_from("<IIII", a.plan, 0)[2:]
    off = 16 + 24 * nslots
    ops = []
    for _ in range(nsteps):
        op, plen = struct.unpack_from("<II", a.plan, off)
        ops.append(op)
        off += 200 + ((plen + 7) // 8) * 8
    assert ops.count(OP_SOFTMAX) == 2 and ops.count(OP_CE_INDEX) == 1
    assert OP_ROW_REDUCE in ops and OP_REDUCE_ALL in ops


def test_unadmitted_node_is_rejected():
    part = Partition({"x": f32(4, 4), "y": T("FLOAT64", (4, 4))},
                     [Node("TANH", ["x"], "y")], ["x"], ["y"])
    with pytest.raises(UnsupportedPartition):
        HipPartitionPreparer().analyze(part)
