"""Reference provider for operators' reference() (test infrastructure).

Maps each operator class to its CPU oracle (oracle/ops.py), so that
OperatorSequence's compare and reference dispatch modes, and op.reference(),
work in the tests. Registered by conftest.py for the whole session.
"""

import torch

from oracle import ops


def reference(op, *inputs):
    name = type(op).__name__
    if name == "GEMV":
        A, x = inputs
        y = ops.gemv_reference(A, x, out_dtype=torch.float32)
        if op.epilogue == "gelu":
            y = ops.gelu_tanh(y.to(torch.bfloat16).float())
        return y.to(torch.bfloat16)
    if name == "SiLU":
        return ops.silu_reference(inputs[0])
    if name == "ElementwiseMul":
        return ops.mul_reference(*inputs)
    if name == "ElementwiseAdd":
        return ops.add_reference(*inputs)
    if name == "GEMM":
        A, B = inputs
        return ops.gemm_reference(A, B, b_col_maj=op.b_col_maj, c_col_maj=op.c_col_maj)
    if name == "RMSNorm":
        x = inputs[0].reshape(-1, op.tile_size)
        w = inputs[1] if len(inputs) > 1 else None
        return ops.rms_norm_reference(x, w, eps=op.epsilon).reshape(-1)
    if name == "Softmax":
        valid = op.rtp_vector_size
        return ops.softmax_reference(inputs[0].reshape(op.rows, op.cols), valid).reshape(-1)
    if name == "GEMVInt4":
        codes, scales, x = inputs
        return ops.gemv_int4_reference(codes, scales, x, signed=op.signed)
    raise NotImplementedError(f"no oracle for {name}")
