"""SwiGLUDecode (iron/operators/swiglu_decode/op.py:13-70): the single-token
SwiGLU feed-forward ``W_down @ (SiLU(W_gate @ x) * (W_up @ x))`` as an
OperatorSequence.

Same runlist and buffer names as the reference: input ``in``; weight buffers
``w_gate`` / ``w_up`` (hidden, embedding) and ``w_down`` (embedding, hidden),
row-major as the GEMV takes them; intermediates ``left``, ``right``,
``left_swished``, ``intermediate``; output ``out``. One GEMV operator serves
both the gate and the up projection. With the default dispatch the five
steps are one captured hipGraph.
"""

from ...common.sequence import OperatorSequence
from ..elementwise_mul.op import ElementwiseMul
from ..gemv.op import GEMV
from ..silu.op import SiLU

N_COLS = 8  # AIE column count the reference derives from the device; a sizing hint here


class SwiGLUDecode(OperatorSequence):
    def __init__(self, embedding_dim, hidden_dim, prio_accuracy=False, context=None, dispatch="auto"):
        self.hidden_dim = hidden_dim
        self.embedding_dim = embedding_dim
        self.prio_accuracy = prio_accuracy
        n = N_COLS
        gemv_1 = GEMV(M=hidden_dim, K=embedding_dim, num_aie_columns=n, tile_size_input=4,
                      tile_size_output=hidden_dim // n, context=context)
        silu = SiLU(size=hidden_dim, num_aie_columns=n, tile_size=hidden_dim // (n * 2), context=context)
        eltwise_mul = ElementwiseMul(size=hidden_dim, num_aie_columns=n, tile_size=hidden_dim // n, context=context)
        gemv_2 = GEMV(M=embedding_dim, K=hidden_dim, num_aie_columns=n, tile_size_input=1,
                      tile_size_output=embedding_dim // n, context=context)
        runlist = [
            (gemv_1, "w_gate", "in", "left"),
            (gemv_1, "w_up", "in", "right"),
            (silu, "left", "left_swished"),
            (eltwise_mul, "left_swished", "right", "intermediate"),
            (gemv_2, "w_down", "intermediate", "out"),
        ]
        super().__init__(
            name=f"swiglu_decode_e{embedding_dim}_h{hidden_dim}",
            runlist=runlist,
            input_args=["in"],
            output_args=["out"],
            dispatch=dispatch,
            context=context,
        )
