"""Small helpers for GPU parity tests: run a one-off program through the C ABI."""
import numpy as np

from synaptik_amd.native import HipProgram
from synaptik_amd.program import NP_DTYPES


def run_program(ctx, builder, inputs, output_slots):
    """inputs: list of numpy arrays in input-index order; returns numpy arrays per output slot."""
    prog = HipProgram(ctx, builder.image())
    in_bufs = [ctx.upload(np.ascontiguousarray(a)) for a in inputs]
    out_bufs = [ctx.buffer(s.nbytes) for s in output_slots]
    prog.run(in_bufs, out_bufs)
    res = [b.download(NP_DTYPES[s.dtype], s.count) for b, s in zip(out_bufs, output_slots)]
    prog.close()
    return res
