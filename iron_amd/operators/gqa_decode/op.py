"""GQADecode: one decode step of grouped-query attention (new fused operator).

Replaces the per-token attention runlist of the reference decode step
(iron/applications/llama_3.2_1b/llama_npu.py:486-523: RoPE q/k, StridedCopy
into the KV cache, Repeat K/V, batched GEMV scores, scale Mul, masked
Softmax, Transpose V, batched GEMV context) with one split-K flash-decode
kernel (iron_gqa_decode); semantics are the CPU golden's
(llama_cpu.py:49-148).

Arg spec: q (H, D), k_new (Hkv, D), v_new (Hkv, D), k_cache and v_cache
(Hkv, max_len, D) inout, angles (angle_rows, D) fp32 [cos, sin] interleaved,
out (H, D). The position comes from ``set_position(pos)`` (host int) or
``position_tensor`` (a device int32 read at run time, for graph replay);
inside an OperatorSequence, ``position_parameter`` names the runtime
parameter that supplies it.
The workspace is allocated by the operator (zeroed once) per device.
"""

import math
from dataclasses import dataclass, field

import torch

from ... import _lib
from ...common import HIPOperator, AIERuntimeArgSpec


@dataclass
class GQADecode(HIPOperator):
    num_heads: int
    num_kv_heads: int
    head_dim: int
    max_len: int
    angle_rows: int | None = None
    scale: float | None = field(default=None, repr=False)
    position_parameter: str | None = field(default=None, repr=False)
    context: object = field(default=None, repr=False)
    # bytes of the per-call device phase trace (iron_amd/common/tracing_utils.py); None: IRON_TRACE_SIZE
    trace_size: int | None = field(default=None, repr=False)

    def __post_init__(self):
        if self.head_dim != 64:
            raise ValueError(f"Only head_dim=64 is supported, got {self.head_dim}")
        if self.num_heads % self.num_kv_heads:
            raise ValueError("num_heads must be a multiple of num_kv_heads")
        if self.num_heads // self.num_kv_heads not in (1, 2, 4, 8):
            raise ValueError("group size num_heads/num_kv_heads must be 1, 2, 4 or 8")
        if self.angle_rows is None:
            self.angle_rows = self.max_len
        if self.scale is None:
            self.scale = 1.0 / math.sqrt(self.head_dim)
        self.position = 0
        self.position_tensor = None
        self._ws = {}
        HIPOperator.__init__(self, context=self.context)

    def set_position(self, pos: int) -> None:
        if not 0 <= pos < min(self.max_len, self.angle_rows):
            raise ValueError(f"position {pos} outside [0, {min(self.max_len, self.angle_rows)})")
        self.position = int(pos)

    def workspace_bytes(self) -> int:
        return int(_lib.query("iron_gqa_decode_workspace_bytes", self.num_heads, self.num_kv_heads,
                              self.head_dim, self.max_len))

    def workspace(self, device) -> torch.Tensor:
        ws = self._ws.get(device)
        if ws is None:
            ws = torch.zeros(self.workspace_bytes(), dtype=torch.uint8, device=device)
            self._ws[device] = ws
        return ws

    def get_arg_spec(self):
        H, Hk, D = self.num_heads, self.num_kv_heads, self.head_dim
        return [
            AIERuntimeArgSpec("in", (H, D)),
            AIERuntimeArgSpec("in", (Hk, D)),
            AIERuntimeArgSpec("in", (Hk, D)),
            AIERuntimeArgSpec("inout", (Hk, self.max_len, D)),
            AIERuntimeArgSpec("inout", (Hk, self.max_len, D)),
            AIERuntimeArgSpec("in", (self.angle_rows, D), dtype=torch.float32),
            AIERuntimeArgSpec("out", (H, D)),
        ]

    def _launch(self, q, k_new, v_new, k_cache, v_cache, angles, out, *, stream):
        ws = self.workspace(q.device)
        _lib.call("iron_gqa_decode", q.data_ptr(), k_new.data_ptr(), v_new.data_ptr(), k_cache.data_ptr(),
                  v_cache.data_ptr(), angles.data_ptr(), self.angle_rows, out.data_ptr(), ws.data_ptr(),
                  self.num_heads, self.num_kv_heads, self.head_dim, self.max_len, self.position,
                  _lib.ptr(self.position_tensor), float(self.scale), stream)
