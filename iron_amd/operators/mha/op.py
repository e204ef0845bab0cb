"""MHA (iron/operators/mha/op.py:21-135): causal multi-head / grouped-query
attention at prefill (S_q = S_kv = seq_len), d = 64.

Arg spec as the reference: Q and O ``(heads*S_pad*d,)``, K and V
``(kv_heads*S_pad*d,)`` with S padded to a multiple of 64*num_of_pipelines;
``num_KV_heads == 0`` means plain MHA. Head h attends KV head
h // (heads / kv_heads). Rows beyond seq_len are written as zeros, matching
the padded golden (mha/reference.py:83-94). Kernel: iron_attention_prefill
(flash attention, fp32 online softmax).
"""

import math
from dataclasses import dataclass, field
from typing import ClassVar, Dict

from ... import _lib
from ...common import HIPOperator, AIERuntimeArgSpec


@dataclass
class MHA(HIPOperator):
    num_heads: int
    seq_len: int
    d: int
    num_KV_heads: int
    num_of_pipelines: int = field(default=1, repr=False)
    context: object = field(default=None, repr=False)

    _name_aliases: ClassVar[Dict[str, str]] = {
        **HIPOperator._name_aliases,
        "num_heads": "h",
        "num_KV_heads": "kv",
        "seq_len": "s",
    }

    def __post_init__(self):
        self.B_q = 64
        self.B_kv = 64
        if self.d != 64:
            raise ValueError(f"Only d=64 is supported in this version, got d={self.d}")
        kv = self.num_KV_heads if self.num_KV_heads else self.num_heads
        if self.num_heads % kv:
            raise ValueError(f"num_heads ({self.num_heads}) must be a multiple of num_KV_heads ({kv})")
        HIPOperator.__init__(self, context=self.context)

    @property
    def seq_padded(self) -> int:
        npipe = self.num_of_pipelines
        return ((self.seq_len + 63 * npipe) // (64 * npipe)) * (64 * npipe)

    def get_arg_spec(self):
        kv = self.num_KV_heads if self.num_KV_heads else self.num_heads
        q_size = self.num_heads * self.d * self.seq_padded
        kv_size = kv * self.d * self.seq_padded
        return [
            AIERuntimeArgSpec("in", (q_size,)),  # Q
            AIERuntimeArgSpec("in", (kv_size,)),  # K
            AIERuntimeArgSpec("in", (kv_size,)),  # V
            AIERuntimeArgSpec("out", (q_size,)),  # O
        ]

    def _launch(self, Q, K, V, O, *, stream):
        kv = self.num_KV_heads if self.num_KV_heads else self.num_heads
        sp, d = self.seq_padded, self.d
        _lib.call("iron_attention_prefill", Q.data_ptr(), K.data_ptr(), V.data_ptr(), O.data_ptr(),
                  self.num_heads, kv, self.seq_len, self.seq_len, d,
                  sp * d, d, sp * d, d, sp * d, d, sp, 1, 0, 1.0 / math.sqrt(d), stream)
