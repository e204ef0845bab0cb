"""Llama-3.2-1B on MI355X: the reference application's forward pass
(iron/applications/llama_3.2_1b/llama_npu.py) rebuilt on the HIP kernels.

Decode (one token) is 6 kernels per layer plus 2, all reading the token id and
position from device memory:

    token = argmax(keys); pos += 1; x = emb[token]       iron_argmax_select
    per layer:
      qkv = Wqkv' . x * inv_rms(x)                       iron_gemv_i4g32_fused (norm fused)
      attn = gqa(rope(q), rope(k) -> cache, v -> cache)  iron_gqa_decode (split-K + merge)
      x  += Wo . attn                                    iron_gemv_i4g32_fused (residual fused)
      h   = silu(Wg' . x * r) * (Wu' . x * r)            iron_gemv_i4g32_fused (pair + norm)
      x  += Wd . h                                       iron_gemv_i4g32_fused (residual fused)
    logits = Whead' . x * inv_rms(x), argmax keys        iron_gemv_bf16_fused

so the step is captured once as a HIP graph and replayed for every token with
no host synchronisation (the reference's single fused decode dispatch,
llama_npu.py:459-584, is the analogue). Each RMSNorm weight is folded into the
columns of the matrix that consumes the normalised vector (W' = W diag(w)),
so the GEMVs only scale their outputs by rsqrt(mean(x^2) + eps). Prefill runs the same layers on bf16
MFMA GEMMs over the prompt (iron_gemm_bf16_nt) with causal flash attention
(iron_attention_prefill), replacing the reference's GEMM + CPU-softmax path
(llama_npu.py:1028-1149).

Weights: every linear layer is quantised once to int4 group-32
(iron_quantize_i4g32). Decode streams the int4 codes; prefill uses bf16
copies produced by dequantising those same codes (iron_dequant_i4), so both
phases compute with identical effective weights. The tied embedding / LM
head stays bf16 (optionally int4 with ``head_int4``).
"""

from __future__ import annotations

import math
from dataclasses import dataclass, field

import torch

from ... import _lib
from ...common.graph import capture_graph

BF16 = torch.bfloat16
KV_RESIDENT = 1  # IRON_GQA_KV_RESIDENT of iron_gqa_decode_ex (include/iron_hip.h)
COUNTERS_ZERO = 2  # IRON_GQA_COUNTERS_ZERO: the workspace's arrival counters are kept at zero


@dataclass
class LlamaConfig:
    """Model constants of llama_inference_harness.py:31-41 plus the KV capacity."""

    vocab_size: int = 128256
    emb_dim: int = 2048
    n_layers: int = 16
    n_heads: int = 32
    n_kv_groups: int = 8
    hidden_dim: int = 8192
    rope_base: float = 500000.0
    rope_scaling: dict | None = field(
        default_factory=lambda: {"factor": 32.0, "low_freq_factor": 1.0, "high_freq_factor": 4.0,
                                 "original_context_length": 8192}
    )
    eps: float = 1e-5
    max_seq_len: int = 4608
    int4: bool = True
    head_int4: bool = False
    # prefill GEMMs dequantise the int4 weights in the kernel instead of
    # keeping bf16 copies (bit-identical results, ~1.7 GB less memory)
    prefill_int4: bool = False
    # split-K prefill GEMMs leave their fp32 partial sums to the next kernel
    # (RoPE scatter, RMSNorm), which merges them: one launch fewer per split
    # GEMM, bit-identical results
    prefill_fuse_merge: bool = True
    # decode step as one launch (iron_llama_decode_fused) plus the head, for the
    # Llama-3.2-1B shape with int4 linears; otherwise (or False) 82 launches
    decode_fused: bool = False
    # bound on every wait inside the one-launch step (microseconds)
    decode_wait_us: int = 200000

    @property
    def head_dim(self) -> int:
        return self.emb_dim // self.n_heads

    @property
    def qkv_dim(self) -> int:
        return (self.n_heads + 2 * self.n_kv_groups) * self.head_dim

    def validate(self) -> None:
        if self.head_dim != 64:
            raise ValueError(f"head_dim must be 64 (emb_dim / n_heads = {self.head_dim})")
        if self.n_heads % self.n_kv_groups or self.n_heads // self.n_kv_groups not in (1, 2, 4, 8):
            raise ValueError("n_heads / n_kv_groups must be 1, 2, 4 or 8")
        if self.emb_dim % 64 or self.hidden_dim % 64:
            raise ValueError("emb_dim and hidden_dim must be multiples of 64")


def compute_rope_angles(head_dim: int, context_length: int, base: float, scaling: dict | None) -> torch.Tensor:
    """fp32 table (context_length, head_dim) of interleaved [cos, sin] pairs.

    The layout of llama_inference_harness.py:109-123; inverse frequencies with
    the llama3 band scaling of iron/operators/rope/reference.py:26-52 when
    ``scaling`` is given (BASELINE: factor 32, low 1, high 4, original 8192).
    """
    inv = 1.0 / (base ** (torch.arange(0, head_dim, 2, dtype=torch.float32) / head_dim))
    if scaling is not None:
        lo_wl = scaling["original_context_length"] / scaling["low_freq_factor"]
        hi_wl = scaling["original_context_length"] / scaling["high_freq_factor"]
        wl = 2 * math.pi / inv
        scaled = torch.where(wl > lo_wl, inv / scaling["factor"], inv)
        smooth = (scaling["original_context_length"] / wl - scaling["low_freq_factor"]) / (
            scaling["high_freq_factor"] - scaling["low_freq_factor"]
        )
        blended = (1 - smooth) * inv / scaling["factor"] + smooth * inv
        inv = torch.where((wl <= lo_wl) & (wl >= hi_wl), blended, scaled)
    ang = torch.outer(torch.arange(context_length, dtype=torch.float32), inv)
    table = torch.empty(context_length, head_dim, dtype=torch.float32)
    table[:, 0::2] = torch.cos(ang)
    table[:, 1::2] = torch.sin(ang)
    return table


def random_weights(cfg: LlamaConfig, device, seed: int = 0, std: float = 0.02) -> dict:
    """Random-init Llama-shaped weights (Hugging Face names, bf16, on ``device``):
    linear and embedding weights ~N(0, std^2), norm weights ~N(1, 0.1^2)."""
    g = torch.Generator(device=device)
    g.manual_seed(seed)

    def normal(*shape, mean=0.0, s=std):
        return (torch.randn(*shape, generator=g, device=device) * s + mean).to(BF16)

    E, H, Hd = cfg.emb_dim, cfg.hidden_dim, cfg.head_dim
    w = {"model.embed_tokens.weight": normal(cfg.vocab_size, E), "model.norm.weight": normal(E, mean=1.0, s=0.1)}
    for i in range(cfg.n_layers):
        p = f"model.layers.{i}."
        w[p + "input_layernorm.weight"] = normal(E, mean=1.0, s=0.1)
        w[p + "post_attention_layernorm.weight"] = normal(E, mean=1.0, s=0.1)
        w[p + "self_attn.q_proj.weight"] = normal(cfg.n_heads * Hd, E)
        w[p + "self_attn.k_proj.weight"] = normal(cfg.n_kv_groups * Hd, E)
        w[p + "self_attn.v_proj.weight"] = normal(cfg.n_kv_groups * Hd, E)
        w[p + "self_attn.o_proj.weight"] = normal(E, cfg.n_heads * Hd)
        w[p + "mlp.gate_proj.weight"] = normal(H, E)
        w[p + "mlp.up_proj.weight"] = normal(H, E)
        w[p + "mlp.down_proj.weight"] = normal(E, H)
    return w


class Linear:
    """One linear layer (out_features, in_features) held as int4-g32 codes +
    scales for decode, plus (unless ``keep_bf16`` is False) the matching
    dequantised bf16 matrix for prefill. Without the copy, prefill GEMMs
    dequantise the int4 weights in the kernel (iron_gemm_i4g32_nt), with
    bit-identical results."""

    def __init__(self, weight: torch.Tensor, int4: bool, stream: int, keep_bf16: bool = True):
        self.N, self.K = weight.shape
        dev = weight.device
        self._bf16 = None
        if int4:
            if self.K % 32:
                raise ValueError(f"in_features {self.K} must be a multiple of 32 for int4")
            self.codes = torch.empty(self.N, self.K // 2, dtype=torch.uint8, device=dev)
            self.scales = torch.empty(self.N, self.K // 32, dtype=BF16, device=dev)
            w = weight.contiguous()
            _lib.call("iron_quantize_i4g32", w.data_ptr(), self.codes.data_ptr(), self.scales.data_ptr(), self.N,
                      self.K, stream)
            if keep_bf16 or self.K % 64:
                self._bf16 = self._dequantized(stream)
        else:
            self.codes = self.scales = None
            self._bf16 = weight.contiguous()
        self.int4 = int4

    def _dequantized(self, stream) -> torch.Tensor:
        out = torch.empty(self.N, self.K, dtype=BF16, device=self.codes.device)
        _lib.call("iron_dequant_i4", self.codes.data_ptr(), self.scales.data_ptr(), out.data_ptr(), self.N, self.K, 32,
                  1, stream)
        return out

    @property
    def bf16(self) -> torch.Tensor:
        """The bf16 matrix (dequantised on demand when no copy is kept)."""
        if self._bf16 is None:
            return self._dequantized(_lib.stream_handle(self.codes.device))
        return self._bf16

    def gemv(self, x, y, stream, norm_scale=False, eps=0.0, residual=None, pair: "Linear | None" = None,
             keys=None):
        """y = [silu](W . x * r) [* (W2 . x * r)] [+ residual] on one token, with
        r = rsqrt(mean(x^2) + eps) when norm_scale (norm weight folded into W)."""
        mode = 2 if norm_scale else 0
        if self.int4:
            _lib.call("iron_gemv_i4g32_fused", self.codes.data_ptr(), self.scales.data_ptr(),
                      _lib.ptr(pair.codes if pair else None), _lib.ptr(pair.scales if pair else None), x.data_ptr(),
                      y.data_ptr(), self.N, self.K, 1, mode, None, float(eps), _lib.ptr(residual), 0, _lib.ptr(keys),
                      stream)
        else:
            _lib.call("iron_gemv_bf16_fused", self._bf16.data_ptr(), _lib.ptr(pair._bf16 if pair else None),
                      x.data_ptr(), y.data_ptr(), self.N, self.K, mode, None, float(eps), _lib.ptr(residual), 0,
                      _lib.ptr(keys), stream)

    def _splits(self, rows):
        """The library's K split for this projection at `rows` rows: the bf16
        policy for a bf16 copy, the int4-g32 one when the GEMM reads the codes."""
        q = "iron_gemm_splitk_choose" if self._bf16 is not None else "iron_gemm_i4g32_splitk_choose"
        return _lib.query(q, rows, self.N, self.K)

    def gemm(self, X, Y, rows, stream, workspace=None):
        """Y (rows, N) = X (rows, K) . W^T on bf16 MFMA; split over K (fp32
        partials in ``workspace(nbytes)``) when the output tiles alone cannot
        fill the GPU. Reads the int4 weights directly when no bf16 copy is kept."""
        splits = self._splits(rows) if workspace is not None else 1
        need, ws = 0, None
        if splits > 1:
            need = int(_lib.query("iron_gemm_splitk_workspace_bytes", rows, self.N, splits))
            ws = workspace(need)
        if self._bf16 is None:
            _lib.call("iron_gemm_i4g32_nt", X.data_ptr(), self.codes.data_ptr(), self.scales.data_ptr(), Y.data_ptr(),
                      rows, self.N, self.K, self.N, 0, 0, 0.0, 0.0, 1, splits, _lib.ptr(ws), need, stream)
        elif splits > 1:
            _lib.call("iron_gemm_bf16_nt_splitk", X.data_ptr(), self._bf16.data_ptr(), Y.data_ptr(), rows, self.N,
                      self.K, self.N, 0, 0, 0.0, 0.0, splits, ws.data_ptr(), need, stream)
        else:
            _lib.call("iron_gemm_bf16_nt", X.data_ptr(), self._bf16.data_ptr(), Y.data_ptr(), rows, self.N, self.K,
                      self.N, 0, 0, 0.0, 0.0, stream)


    def gemm_partials(self, X, rows, stream, workspace):
        """The first pass of the split-K GEMM alone: fp32 partial sums of X . W^T,
        (splits, rows, N) in ``workspace(nbytes)``, for a consumer that merges
        them (iron_rmsnorm_splitk, iron_qkv_rope_scatter_splitk). Returns
        (partials, splits), or None when this shape is not split (use gemm)."""
        splits = self._splits(rows)
        if splits < 2:
            return None
        need = int(_lib.query("iron_gemm_splitk_workspace_bytes", rows, self.N, splits))
        ws = workspace(need)
        i4 = self._bf16 is None
        _lib.call("iron_gemm_nt_partials", X.data_ptr(), _lib.ptr(None if i4 else self._bf16),
                  _lib.ptr(self.codes if i4 else None), _lib.ptr(self.scales if i4 else None), 1, rows, self.N,
                  self.K, splits, ws.data_ptr(), need, stream)
        return ws, splits


class LlamaHIP:
    """Llama-3.2-1B-shaped model on one GPU: weights, KV caches and the decode graph."""

    MAX_PREFILL_GRAPHS = 16  # captured prefill shapes kept at once (least recently used dropped first)

    def __init__(self, cfg: LlamaConfig, weights: dict, device=None):
        cfg.validate()
        self.cfg = cfg
        self.device = torch.device(device) if device is not None else torch.device("cuda", 0)
        _lib.load()
        s = self._stream()
        E, Hd = cfg.emb_dim, cfg.head_dim
        dev = self.device
        w = {k: v.to(dev, BF16).contiguous() for k, v in weights.items()}

        def fold(W, norm):  # W diag(norm): the norm weight moves into the matrix columns
            return (W.float() * norm.float().unsqueeze(0)).to(BF16)

        self.embed = w["model.embed_tokens.weight"]
        self.final_norm = w["model.norm.weight"]
        # tied head (the reference's model) unless the weights carry their own lm_head
        self.head = Linear(fold(w.get("lm_head.weight", self.embed), self.final_norm), cfg.head_int4, s)
        self.layers = []
        keep = not cfg.prefill_int4
        for i in range(cfg.n_layers):
            p = f"model.layers.{i}."
            an, fn = w[p + "input_layernorm.weight"], w[p + "post_attention_layernorm.weight"]
            qkv = torch.cat([w[p + "self_attn.q_proj.weight"], w[p + "self_attn.k_proj.weight"],
                             w[p + "self_attn.v_proj.weight"]], dim=0)
            self.layers.append({
                "attn_norm": an,
                "ffn_norm": fn,
                "qkv": Linear(fold(qkv, an), cfg.int4, s, keep_bf16=keep),
                "o": Linear(w[p + "self_attn.o_proj.weight"], cfg.int4, s, keep_bf16=keep),
                "gate": Linear(fold(w[p + "mlp.gate_proj.weight"], fn), cfg.int4, s, keep_bf16=keep),
                "up": Linear(fold(w[p + "mlp.up_proj.weight"], fn), cfg.int4, s, keep_bf16=keep),
                "down": Linear(w[p + "mlp.down_proj.weight"], cfg.int4, s, keep_bf16=keep),
            })
            if keep:  # prefill SwiGLU as one GEMM over 64-row blocks alternating gate / up
                L = self.layers[-1]
                F, K = L["gate"].N, L["gate"].K
                L["gate_up"] = torch.stack([L["gate"].bf16.view(F // 64, 64, K), L["up"].bf16.view(F // 64, 64, K)],
                                           dim=1).reshape(2 * F, K).contiguous()
                if cfg.int4:  # the decode GEMVs read the int4 codes; the separate copies are not needed
                    L["gate"]._bf16 = L["up"]._bf16 = None
        del w
        L = cfg.max_seq_len
        self.k_cache = [torch.zeros(cfg.n_kv_groups, L, Hd, dtype=BF16, device=dev) for _ in range(cfg.n_layers)]
        self.v_cache = [torch.zeros(cfg.n_kv_groups, L, Hd, dtype=BF16, device=dev) for _ in range(cfg.n_layers)]
        self.angles = compute_rope_angles(Hd, L, cfg.rope_base, cfg.rope_scaling).to(dev)
        ws = _lib.query("iron_gqa_decode_workspace_bytes", cfg.n_heads, cfg.n_kv_groups, Hd, L)
        self.attn_ws = torch.zeros(int(ws), dtype=torch.uint8, device=dev)
        # The decode step reads every layer's caches once per token while ~1 GB of
        # weights streams past them: caches that fit well inside the 256 MB
        # Infinity Cache stay there between steps when the attention reads them
        # with allocating loads (IRON_GQA_KV_RESIDENT).
        kv_bytes = 2 * cfg.n_layers * cfg.n_kv_groups * L * Hd * 2
        self.kv_flags = KV_RESIDENT if kv_bytes <= (192 << 20) else 0
        # decode buffers (fixed addresses: the captured graph refers to them)
        self.x = torch.zeros(E, dtype=BF16, device=dev)
        self.qkv = torch.zeros(cfg.qkv_dim, dtype=BF16, device=dev)
        self.attn = torch.zeros(cfg.n_heads * Hd, dtype=BF16, device=dev)
        self.h = torch.zeros(cfg.hidden_dim, dtype=BF16, device=dev)
        self.logits = torch.zeros(cfg.vocab_size, dtype=BF16, device=dev)
        self.xn = torch.zeros(E, dtype=BF16, device=dev)
        self.token = torch.zeros(1, dtype=torch.int32, device=dev)
        self.n_keys = (cfg.vocab_size + 3) // 4
        self.keys = torch.zeros(self.n_keys, dtype=torch.int64, device=dev)
        self.pos = torch.zeros(1, dtype=torch.int32, device=dev)
        self.history = torch.zeros(L, dtype=torch.int32, device=dev)
        self.host_pos = 0
        # The one-launch decode step (Llama-3.2-1B shape, int4 linears): a device
        # table of per-layer pointers (IronDecodeLayer), the exchange area, the
        # epoch its tags carry and the status word its bounded waits report to.
        self.fused = bool(cfg.decode_fused and cfg.int4 and cfg.emb_dim == 2048 and cfg.hidden_dim == 8192
                          and cfg.n_heads == 32 and cfg.n_kv_groups == 8 and cfg.max_seq_len % 64 == 0
                          and cfg.max_seq_len <= 6144 and _lib.query("iron_xcd_round_robin", s) == 1)
        if self.fused:
            table = []
            for i, Ly in enumerate(self.layers):
                for name in ("qkv", "o", "gate", "up", "down"):
                    table += [Ly[name].codes.data_ptr(), Ly[name].scales.data_ptr()]
                table += [self.k_cache[i].data_ptr(), self.v_cache[i].data_ptr()]
            self.layer_table = torch.tensor(table, dtype=torch.int64).to(dev)
            nbytes = int(_lib.query("iron_llama_decode_fused_exchange_bytes", cfg.n_layers))
            self.exchange = torch.zeros(nbytes, dtype=torch.uint8, device=dev)
            self.epoch = torch.ones(1, dtype=torch.int32, device=dev)
            self.status = torch.zeros(1, dtype=torch.int32, device=dev)
        self.graph = None  # attention chunk positions -> one-step decode graph
        self.graph_multi = None  # attention chunk positions -> DECODE_GRAPH_STEPS-step graph
        self._prefill_bufs = None  # activations of the longest prompt seen (see _pbufs)
        self._prefill_graphs = {}  # (prompt length, start position) -> captured prefill, least recently used first
        self._gemm_ws = torch.empty(0, dtype=torch.uint8, device=dev)
        torch.cuda.synchronize(dev)

    # ------------------------------------------------------------ helpers
    def _stream(self) -> int:
        return _lib.stream_handle(self.device)

    def effective_weights(self) -> dict:
        """Weights the model computes with, as fp32 in the reference's layout (HF
        names): the int4-g32 dequantised matrices with the folded norm weights
        divided back out, the norms, and an untied ``lm_head.weight``."""
        cfg = self.cfg
        q_rows, kv_rows = cfg.n_heads * cfg.head_dim, cfg.n_kv_groups * cfg.head_dim

        def unfold(W, norm):
            return W.float() / norm.float().unsqueeze(0)

        out = {"model.embed_tokens.weight": self.embed.float(), "model.norm.weight": self.final_norm.float(),
               "lm_head.weight": unfold(self.head.bf16, self.final_norm)}
        for i, L in enumerate(self.layers):
            p = f"model.layers.{i}."
            qkv = unfold(L["qkv"].bf16, L["attn_norm"])
            out[p + "self_attn.q_proj.weight"] = qkv[:q_rows]
            out[p + "self_attn.k_proj.weight"] = qkv[q_rows : q_rows + kv_rows]
            out[p + "self_attn.v_proj.weight"] = qkv[q_rows + kv_rows :]
            out[p + "self_attn.o_proj.weight"] = L["o"].bf16.float()
            out[p + "mlp.gate_proj.weight"] = unfold(L["gate"].bf16, L["ffn_norm"])
            out[p + "mlp.up_proj.weight"] = unfold(L["up"].bf16, L["ffn_norm"])
            out[p + "mlp.down_proj.weight"] = L["down"].bf16.float()
            out[p + "input_layernorm.weight"] = L["attn_norm"].float()
            out[p + "post_attention_layernorm.weight"] = L["ffn_norm"].float()
        return out

    def reset(self) -> None:
        """Empty the KV cache (positions restart at 0); cache contents need no clearing."""
        self.host_pos = 0
        self.pos.copy_(torch.zeros(1, dtype=torch.int32))

    # ------------------------------------------------------------ decode
    def _chunk_positions(self, pos: int) -> int:
        """Positions per attention chunk the decode attention takes at `pos` (64
        or 128: its launch shape, chosen from a position hint; 64 for the
        one-launch step, whose attention is its own)."""
        cfg = self.cfg
        if self.fused:
            return 64
        return int(_lib.query("iron_gqa_decode_chunk_positions_ex", cfg.n_heads, cfg.n_kv_groups, cfg.head_dim,
                              cfg.max_seq_len, pos, self.kv_flags, self._stream()))

    def _decode_shapes(self) -> dict:
        """One position hint per attention launch shape the decode can take
        (the shape depends on the position, which the graphs keep on the device)."""
        shapes = {}
        for p in (0, self.cfg.max_seq_len - 1):
            shapes.setdefault(self._chunk_positions(p), p)
        return shapes

    def decode_step(self, pos_hint: int = -1) -> None:
        """Enqueue one decode step: the previous step's argmax keys pick the token
        (pos advances), then the layers, then the head writes logits and keys.
        pos_hint: the position the step is expected at (it picks the attention's
        launch shape only; the position itself is read on the device)."""
        cfg, s = self.cfg, self._stream()
        Hd, q_rows, kv_rows = cfg.head_dim, cfg.n_heads * cfg.head_dim, cfg.n_kv_groups * cfg.head_dim
        if self.fused:
            _lib.call("iron_llama_decode_fused", self.layer_table.data_ptr(), cfg.n_layers, self.keys.data_ptr(),
                      self.n_keys, self.embed.data_ptr(), cfg.vocab_size, self.token.data_ptr(), self.pos.data_ptr(),
                      self.history.data_ptr(), cfg.max_seq_len, self.angles.data_ptr(), self.angles.shape[0],
                      cfg.max_seq_len, 1.0 / math.sqrt(Hd), cfg.eps, self.attn_ws.data_ptr(),
                      self.exchange.data_ptr(), self.x.data_ptr(), self.epoch.data_ptr(), self.status.data_ptr(),
                      cfg.decode_wait_us, self.kv_flags, s)
            h = self.head
            _lib.call("iron_llama_decode_head", _lib.ptr(None if h.int4 else h.bf16), _lib.ptr(h.codes if h.int4 else None),
                      _lib.ptr(h.scales if h.int4 else None), self.x.data_ptr(), self.logits.data_ptr(), h.N, h.K,
                      cfg.eps, self.keys.data_ptr(), self.epoch.data_ptr(), s)
            return
        _lib.call("iron_argmax_select", self.keys.data_ptr(), self.n_keys, self.embed.data_ptr(), cfg.emb_dim,
                  cfg.vocab_size, self.x.data_ptr(), self.token.data_ptr(), self.pos.data_ptr(),
                  self.history.data_ptr(), cfg.max_seq_len, s)
        q = self.qkv[:q_rows]
        k = self.qkv[q_rows : q_rows + kv_rows]
        v = self.qkv[q_rows + kv_rows :]
        scale = 1.0 / math.sqrt(Hd)
        for i, L in enumerate(self.layers):
            L["qkv"].gemv(self.x, self.qkv, s, norm_scale=True, eps=cfg.eps)
            _lib.call("iron_gqa_decode_ex", q.data_ptr(), k.data_ptr(), v.data_ptr(), self.k_cache[i].data_ptr(),
                      self.v_cache[i].data_ptr(), self.angles.data_ptr(), self.angles.shape[0], self.attn.data_ptr(),
                      self.attn_ws.data_ptr(), cfg.n_heads, cfg.n_kv_groups, Hd, cfg.max_seq_len, pos_hint,
                      self.pos.data_ptr(), scale, self.kv_flags | COUNTERS_ZERO, s)
            L["o"].gemv(self.attn, self.x, s, residual=self.x)
            L["gate"].gemv(self.x, self.h, s, norm_scale=True, eps=cfg.eps, pair=L["up"])
            L["down"].gemv(self.h, self.x, s, residual=self.x)
        self.head.gemv(self.x, self.logits, s, norm_scale=True, eps=cfg.eps, keys=self.keys)

    def check_decode_status(self) -> None:
        """Raise if a wait inside a one-launch decode step gave up (waits for the
        stream). The status word is cleared, so later steps can run again."""
        if not self.fused:
            return
        st = int(self.status.item())
        if st:
            # a step that gave up can leave attention arrival counters part-way
            self.attn_ws.zero_()
            self.status.zero_()
            torch.cuda.synchronize(self.device)
            raise RuntimeError(f"one-launch decode step: a wait gave up (status 0x{st:x}; bits: 1 layer input, "
                               "2 position, 4 q/k/v, 8 attention output, 16 o_proj output, 32 h)")

    def commit(self) -> None:
        """Record the token chosen by the last logits (history[pos], pos += 1)
        without starting a step."""
        cfg = self.cfg
        _lib.call("iron_argmax_select", self.keys.data_ptr(), self.n_keys, None, cfg.emb_dim, cfg.vocab_size, None,
                  self.token.data_ptr(), self.pos.data_ptr(), self.history.data_ptr(), cfg.max_seq_len,
                  self._stream())

    def _warmup(self) -> None:
        """Run every decode kernel once eagerly (code objects load before capture).

        Uses the last cache slot, which a later step at that position rewrites
        before any attention reads it; token and position are restored.
        """
        tok, pos, keys = self.token.clone(), self.pos.clone(), self.keys.clone()
        for hint in self._decode_shapes().values():
            self.pos.fill_(self.cfg.max_seq_len - 1)
            self.decode_step(hint)
        self.token.copy_(tok)
        self.pos.copy_(pos)
        self.keys.copy_(keys)
        torch.cuda.synchronize(self.device)
        self.check_decode_status()

    # decode steps per replay of the multi-step graph: fewer graph launches per token
    # (measured at KV 3968 -> 4096: 457.9 us/token with one step per graph, 454.0 with 4, 453.6 with 8)
    DECODE_GRAPH_STEPS = 8

    def capture_decode_graph(self) -> None:
        """Capture decode_step() as HIP graphs: one step, and DECODE_GRAPH_STEPS
        steps back to back (the position advances on the device inside), for
        each attention launch shape the decode can take."""
        self._warmup()
        k = self.DECODE_GRAPH_STEPS
        self.graph, self.graph_multi = {}, {}
        for shape, hint in self._decode_shapes().items():
            self.graph[shape] = capture_graph(lambda: self.decode_step(hint), self.device)
            self.graph_multi[shape] = capture_graph(lambda: [self.decode_step(hint) for _ in range(k)], self.device)

    def decode(self, n_steps: int, use_graph: bool = True) -> None:
        """Run n_steps greedy decode steps from the current token and position
        (with graphs: the multi-step graph while it fits, then single steps)."""
        if self.host_pos + n_steps > self.cfg.max_seq_len:
            raise ValueError(f"decoding {n_steps} steps from position {self.host_pos} exceeds the KV capacity "
                             f"{self.cfg.max_seq_len}")
        if use_graph and self.graph is None:
            self.capture_decode_graph()
        left, pos = n_steps, self.host_pos
        if use_graph:
            k = self.DECODE_GRAPH_STEPS
            while left >= k:
                self.graph_multi[self._chunk_positions(pos + k // 2)].replay()
                left -= k
                pos += k
        for _ in range(left):
            if use_graph:
                self.graph[self._chunk_positions(pos)].replay()
            else:
                self.decode_step(pos)
            pos += 1
        self.host_pos += n_steps
        self.check_decode_status()

    # ------------------------------------------------------------ prefill
    def _drop_prefill_graphs(self) -> None:
        """Forget every captured prefill graph, after the GPU has finished any
        replay of them (destroying an executable graph while it runs is not
        defined). Never called under capture: capture follows an eager run of
        the same shape, which has already sized the workspace and buffers."""
        if self._prefill_graphs:
            if torch.cuda.is_current_stream_capturing():
                raise RuntimeError("prefill buffers or workspace resized during graph capture")
            torch.cuda.synchronize(self.device)
            self._prefill_graphs.clear()

    def _workspace(self, nbytes: int) -> torch.Tensor:
        """Split-K GEMM workspace of at least ``nbytes`` (grown on demand; stream-ordered reuse).
        Growing it drops the captured prefill graphs, which point into the old one."""
        if self._gemm_ws.numel() < nbytes:
            self._drop_prefill_graphs()
            self._gemm_ws = torch.empty(nbytes, dtype=torch.uint8, device=self.device)
        return self._gemm_ws

    def _pbufs(self, S: int):
        """Prefill activations for S tokens: views of one set of buffers sized for
        the longest prompt seen (rounded up to a power of two, at most the KV
        capacity), so memory stays bounded by that prompt whatever lengths
        come and go. Growing them drops the captured prefill graphs."""
        b = self._prefill_bufs
        if b is None or b["cap"] < S:
            cfg, dev = self.cfg, self.device
            E, Hd = cfg.emb_dim, cfg.head_dim
            cap = min(max(64, 1 << (S - 1).bit_length()), max(S, cfg.max_seq_len))
            self._drop_prefill_graphs()
            self._prefill_bufs = None  # release the old set before allocating the new one
            b = {"cap": cap}
            for name, cols, dt in (("ids", 0, torch.int32), ("X", E, BF16), ("Xn", E, BF16),
                                   ("QKV", cfg.qkv_dim, BF16), ("Q", cfg.n_heads * Hd, BF16),
                                   ("O", cfg.n_heads * Hd, BF16), ("T", E, BF16), ("G", cfg.hidden_dim, BF16),
                                   ("U", cfg.hidden_dim, BF16)):
                b[name] = torch.zeros((cap, cols) if cols else (cap,), dtype=dt, device=dev)
            self._prefill_bufs = b
        return {k: (v if k == "cap" else v[:S]) for k, v in b.items()}

    def prefill(self, token_ids, use_graph: bool = False) -> None:
        """Process the prompt at positions pos..pos+S-1; leaves logits of the last
        position in self.logits and the greedy next token in self.token.

        With ``use_graph`` the launches run as a hipGraph captured once per
        (prompt length, start position) -- after one eager run of that shape --
        and replayed afterwards, so the host issues one graph instead of ~150
        kernels. Results are bit-identical to the eager path. At most
        MAX_PREFILL_GRAPHS shapes are kept (least recently used dropped first);
        all are dropped when the split-K workspace or the activation buffers
        they point into are reallocated."""
        cfg = self.cfg
        ids = torch.as_tensor(token_ids, dtype=torch.int32).reshape(-1)
        S = int(ids.numel())
        pos0 = self.host_pos
        if S == 0 or pos0 + S > cfg.max_seq_len:
            raise ValueError(f"prompt of {S} tokens at position {pos0} does not fit the KV capacity {cfg.max_seq_len}")
        b = self._pbufs(S)
        b["ids"].copy_(ids)
        key = (S, pos0)
        graph = self._prefill_graphs.pop(key, None) if use_graph else None
        if graph is not None:
            self._prefill_graphs[key] = graph  # most recently used last
            graph.replay()
        else:
            self._prefill_launches(S, pos0)  # also sizes the workspace and buffers the capture will use
            if use_graph:
                if len(self._prefill_graphs) >= self.MAX_PREFILL_GRAPHS:
                    torch.cuda.synchronize(self.device)  # a replay of the graph dropped below may still run
                    while len(self._prefill_graphs) >= self.MAX_PREFILL_GRAPHS:
                        self._prefill_graphs.pop(next(iter(self._prefill_graphs)))  # least recently used
                self._prefill_graphs[key] = capture_graph(lambda: self._prefill_launches(S, pos0), self.device)
        self.pos.copy_(torch.tensor([pos0 + S - 1], dtype=torch.int32))
        self.host_pos = pos0 + S

    def _prefill_launches(self, S: int, pos0: int) -> None:
        """Every kernel of one prefill of S tokens at pos0 (token ids already in the
        prefill buffer), on the current stream; capturable."""
        cfg, s = self.cfg, self._stream()
        b = self._pbufs(S)
        E, Hd = cfg.emb_dim, cfg.head_dim
        X, Xn, T = b["X"], b["Xn"], b["T"]
        _lib.call("iron_embedding", self.embed.data_ptr(), b["ids"].data_ptr(), X.data_ptr(), S, E, cfg.vocab_size, s)
        scale = 1.0 / math.sqrt(Hd)
        eps = float(cfg.eps)

        def linear(L, Xin, Yout):
            """Yout = Xin . W^T, or None with the split-K partials returned for the next kernel to merge."""
            part = L.gemm_partials(Xin, S, s, self._workspace) if cfg.prefill_fuse_merge else None
            if part is None:
                L.gemm(Xin, Yout, S, s, self._workspace)
            return part

        def add_norm(part):
            """X += T (or the merged partials of the GEMM that produced it); Xn = norm(X)."""
            if part is None:
                _lib.call("iron_rmsnorm", X.data_ptr(), T.data_ptr(), None, Xn.data_ptr(), X.data_ptr(), S, E, eps, s)
            else:
                _lib.call("iron_rmsnorm_splitk", X.data_ptr(), part[0].data_ptr(), part[1], None, Xn.data_ptr(),
                          X.data_ptr(), S, E, eps, s)

        pending = None  # partials of the previous layer's down projection
        for i, L in enumerate(self.layers):
            # norm weights are folded into the next matrices: unweighted RMSNorm
            if i == 0:
                _lib.call("iron_rmsnorm", X.data_ptr(), None, None, Xn.data_ptr(), None, S, E, eps, s)
            else:  # X += previous FFN output, Xn = norm(X)
                add_norm(pending)
            part = linear(L["qkv"], Xn, b["QKV"])
            rope_args = (self.angles.data_ptr(), self.angles.shape[0], b["Q"].data_ptr(), self.k_cache[i].data_ptr(),
                         self.v_cache[i].data_ptr(), S, cfg.n_heads, cfg.n_kv_groups, Hd, cfg.max_seq_len, pos0, s)
            if part is None:
                _lib.call("iron_qkv_rope_scatter", b["QKV"].data_ptr(), *rope_args)
            else:
                _lib.call("iron_qkv_rope_scatter_splitk", part[0].data_ptr(), part[1], *rope_args)
            _lib.call("iron_attention_prefill", b["Q"].data_ptr(), self.k_cache[i].data_ptr(),
                      self.v_cache[i].data_ptr(), b["O"].data_ptr(), cfg.n_heads, cfg.n_kv_groups, S, pos0 + S, Hd,
                      Hd, cfg.n_heads * Hd, cfg.max_seq_len * Hd, Hd, Hd, cfg.n_heads * Hd, S, 1, pos0, scale, s)
            add_norm(linear(L["o"], b["O"], T))
            if "gate_up" in L:  # G = silu(Xn Wg^T) * (Xn Wu^T) in one GEMM
                _lib.call("iron_gemm_bf16_nt_swiglu", Xn.data_ptr(), L["gate_up"].data_ptr(), b["G"].data_ptr(), S,
                          cfg.hidden_dim, E, cfg.hidden_dim, s)
            else:
                L["gate"].gemm(Xn, b["G"], S, s, self._workspace)
                L["up"].gemm(Xn, b["U"], S, s, self._workspace)
                _lib.call("iron_silu_mul", b["G"].data_ptr(), b["U"].data_ptr(), b["G"].data_ptr(),
                          S * cfg.hidden_dim, s)
            pending = linear(L["down"], b["G"], T)
        add_norm(pending)
        self.head.gemv(Xn[S - 1], self.logits, s, keys=self.keys)

    def set_token(self, token: int) -> None:
        """Force the next input token (teacher forcing): the next step's selection
        picks it regardless of the logits."""
        forced = (0xFFFFFFFF << 32) | (0xFFFFFFFF - int(token))  # above every logit's key (unsigned order)
        self.keys[:1].copy_(torch.tensor([forced - (1 << 64)], dtype=torch.int64))  # same bits as int64

    def generate(self, prompt_ids, n_tokens: int, use_graph: bool = True) -> list[int]:
        """Greedy generation: prefill the prompt, then n_tokens-1 decode steps.
        Returns the n_tokens generated ids (read back once at the end)."""
        self.reset()
        self.prefill(prompt_ids)
        S = self.host_pos
        if n_tokens > 1:
            self.decode(n_tokens - 1, use_graph=use_graph)
        self.commit()
        torch.cuda.synchronize(self.device)
        return self.history[S - 1 : S - 1 + n_tokens].tolist()
