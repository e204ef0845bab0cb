"""SwiGLUPrefill (iron/operators/swiglu_prefill/op.py:13-115): the SwiGLU
feed-forward over ``seq_len`` tokens as an OperatorSequence of GEMMs.

Same runlist and buffer names as the reference: input ``in`` (seq_len,
embedding); weights ``w_gate`` / ``w_up`` and ``w_down`` stored (K, N), or
(N, K) when ``b_col_maj`` (the layout the decode GEMV reads, so prefill and
decode can share one weight copy); intermediates ``left``, ``right``,
``left_swished``, ``intermediate``; output ``out`` (seq_len, embedding).
The GEMMs run on MFMA (iron_gemm_bf16_nt); ``prio_accuracy`` is accepted
(bf16 products with fp32 accumulation are what the kernel always does).
"""

from ...common.sequence import OperatorSequence
from ..elementwise_mul.op import ElementwiseMul
from ..gemm.op import GEMM
from ..silu.op import SiLU

N_COLS = 8


class SwiGLUPrefill(OperatorSequence):
    def __init__(self, seq_len, embedding_dim, hidden_dim, prio_accuracy=False, b_col_maj=False, context=None,
                 dispatch="auto"):
        self.seq_len = seq_len
        self.hidden_dim = hidden_dim
        self.embedding_dim = embedding_dim
        self.prio_accuracy = prio_accuracy
        self.b_col_maj = b_col_maj
        n = N_COLS
        gemm_1 = GEMM(M=seq_len, K=embedding_dim, N=hidden_dim, num_aie_columns=n, b_col_maj=b_col_maj,
                      prio_accuracy=prio_accuracy, context=context)
        self.seq_len_aligned = gemm_1.M
        self.embedding_dim_aligned = gemm_1.K
        self.hidden_dim_aligned = gemm_1.N
        size = self.seq_len_aligned * self.hidden_dim_aligned
        silu = SiLU(size=size, num_aie_columns=n, tile_size=self.hidden_dim_aligned // n, context=context)
        eltwise_mul = ElementwiseMul(size=size, num_aie_columns=n, tile_size=self.hidden_dim_aligned // n,
                                     context=context)
        gemm_2 = GEMM(M=seq_len, K=hidden_dim, N=embedding_dim, num_aie_columns=n, b_col_maj=b_col_maj,
                      prio_accuracy=prio_accuracy, context=context)
        runlist = [
            (gemm_1, "in", "w_gate", "left"),
            (gemm_1, "in", "w_up", "right"),
            (silu, "left", "left_swished"),
            (eltwise_mul, "left_swished", "right", "intermediate"),
            (gemm_2, "intermediate", "w_down", "out"),
        ]
        super().__init__(
            name=f"swiglu_prefill_s{seq_len}_e{embedding_dim}_h{hidden_dim}" + ("_bc" if b_col_maj else ""),
            runlist=runlist,
            input_args=["in"],
            output_args=["out"],
            dispatch=dispatch,
            context=context,
        )
