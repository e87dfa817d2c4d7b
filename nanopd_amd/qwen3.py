"""Qwen3 decoder with random weights whose attention runs on the paged
kernels: the caller side of the hot path, as ModelRunner.paged_forward
(nanoPD/engine/model_runner.py:75-213) patches HF Qwen3 attention.

Per layer and per engine step, for a packed ragged batch (prefill chunk
tokens first, then one token per decode sequence):
  RMSNorm -> fused QKV projection -> qk_norm_rope_store (per-head RMSNorm of
  q and k, RoPE at each token's position, K/V into the paged pool by slot,
  one launch) -> paged_prefill_attention for the prefill rows and
  paged_attention_forward for the decode rows -> o_proj + residual ->
  RMSNorm -> SwiGLU MLP + residual.
With fused_prologue=False the prologue runs as PyTorch ops (HF Qwen3RMSNorm
rounding, fp32 rotate-half RoPE) followed by paged_kv_store_slots.
The reference stores K/V first and attends after (model_runner.py:146, :189);
so does this. Its prefill SDPA sees only the chunk (model_runner.py:152-168);
here prefill rows attend to the paged prefix as well, the same result for a
sequence's first chunk and the correct one for later chunks.

GEMMs, norms and activations are PyTorch (rocBLAS / hipBLASLt on the GPU);
the attention backend is a parameter so that a test can run the same model
with a PyTorch restatement of the attention and compare.
Shapes follow Qwen3-8B (config.json of the Qwen3 release): 36 layers, hidden
4096, 32 query / 8 kv heads of 128, MLP 12288, vocab 151936, RoPE theta 1e6,
RMSNorm eps 1e-6, untied LM head.
The reference's runner also serves Qwen2 (and Llama) models
(model_runner.py:53-58) and applies q_norm / k_norm only where the attention
has them (:101-104). Qwen3Config's qk_norm=False, qkv_bias=True and
tie_word_embeddings=True give that layer (Qwen2: q/k/v biases, no q/k norms,
tied LM head on the 1.5B model); the fused prologue then runs without norm
weights.
"""
from __future__ import annotations

import math
from dataclasses import dataclass
from typing import Callable, Optional

import torch
import torch.nn.functional as F

from . import paged_kernels as pk


@dataclass(frozen=True)
class Qwen3Config:
    num_layers: int = 36
    hidden: int = 4096
    num_heads: int = 32
    num_kv_heads: int = 8
    head_dim: int = 128
    intermediate: int = 12288
    vocab: int = 151936
    rope_theta: float = 1.0e6
    rms_eps: float = 1.0e-6
    init_std: float = 0.02
    qk_norm: bool = True              # per-head q/k RMSNorm (Qwen3); False: Qwen2 / Llama
    qkv_bias: bool = False            # q/k/v projection biases (Qwen2)
    tie_word_embeddings: bool = False  # LM head = embedding (Qwen2-1.5B)

    @property
    def num_params(self) -> int:
        width = (self.num_heads + 2 * self.num_kv_heads) * self.head_dim
        qkv = self.hidden * width + (width if self.qkv_bias else 0)
        o = self.num_heads * self.head_dim * self.hidden
        mlp = 3 * self.hidden * self.intermediate
        norms = 2 * self.hidden + (2 * self.head_dim if self.qk_norm else 0)
        heads = (1 if self.tie_word_embeddings else 2) * self.vocab * self.hidden
        return self.num_layers * (qkv + o + mlp + norms) + heads + self.hidden


QWEN3_8B = Qwen3Config()
# Qwen2-1.5B (config.json of the Qwen2 release; configuration 1's head shape)
QWEN2_1_5B = Qwen3Config(num_layers=28, hidden=1536, num_heads=12, num_kv_heads=2, head_dim=128,
                         intermediate=8960, vocab=151936, rope_theta=1.0e6, rms_eps=1.0e-6,
                         qk_norm=False, qkv_bias=True, tie_word_embeddings=True)


@dataclass
class StepBatch:
    """One engine step's packed batch, prefill sequences first.
    meta: pack_metadata output; num_prefill_seqs / num_prefill_tokens: the
    prefill part; sample_rows: token rows whose logits are wanted."""
    input_ids: torch.Tensor          # int64 [T]
    meta: pk.BatchMetadata
    num_prefill_seqs: int
    num_prefill_tokens: int
    sample_rows: Optional[torch.Tensor]   # int64 [R]; None: every row
    max_prefill_q: int = 0           # longest prefill chunk (grid bound)
    decode_workspace: Optional[torch.Tensor] = None   # explicit decode-attention workspace


# attention(layer, q [T,H,D], k_cache, v_cache, batch, out [T,H,D]) -> None
Attention = Callable[[int, torch.Tensor, torch.Tensor, torch.Tensor, StepBatch, torch.Tensor], None]


def _check_kv_dtype(kv_cache_dtype: str) -> None:
    if kv_cache_dtype not in ("auto", "fp8"):
        raise ValueError(f"kv_cache_dtype must be 'auto' or 'fp8', not {kv_cache_dtype!r}")


class PagedQwen3:
    def __init__(self, cfg: Qwen3Config, num_blocks: int, block_size: int = 16,
                 device: str | torch.device = "cuda", dtype: torch.dtype = torch.bfloat16,
                 seed: int = 0, attention: Optional[Attention] = None,
                 fused_prologue: bool = True, kv_cache_dtype: str = "auto",
                 kv_scale: float = 1.0 / 16):
        """kv_cache_dtype "fp8": the K/V pools hold OCP e4m3 bytes with static
        per-(layer, kv head) scales ``kv_scale`` (element = e4m3 * scale; the
        default covers |x| <= 28), written by the fused prologue (or the FP8
        slot store) and read by the FP8 prefill and decode ops. "auto": pools
        in ``dtype``."""
        _check_kv_dtype(kv_cache_dtype)
        self.cfg = cfg
        self.device = torch.device(device)
        self.dtype = dtype
        self.block_size = block_size
        self.num_blocks = num_blocks
        self.scale = 1.0 / math.sqrt(cfg.head_dim)
        self.attention = attention or self._paged_attention
        self.fused_prologue = fused_prologue
        g = torch.Generator(device=self.device)
        g.manual_seed(seed)

        def rnd(*shape):
            w = torch.empty(*shape, dtype=dtype, device=self.device)
            w.normal_(0.0, cfg.init_std, generator=g)
            return w

        def ones(n):
            return torch.ones(n, dtype=dtype, device=self.device)

        H, KV, D, E = cfg.num_heads, cfg.num_kv_heads, cfg.head_dim, cfg.hidden
        self.embed = rnd(cfg.vocab, E)
        self.layers = []
        for _ in range(cfg.num_layers):
            self.layers.append({
                "in_norm": ones(E),
                "qkv": rnd((H + 2 * KV) * D, E),
                "qkv_bias": rnd((H + 2 * KV) * D) if cfg.qkv_bias else None,
                "q_norm": ones(D) if cfg.qk_norm else None,
                "k_norm": ones(D) if cfg.qk_norm else None,
                "o": rnd(E, H * D),
                "post_norm": ones(E),
                "gate_up": rnd(2 * cfg.intermediate, E),
                "down": rnd(E, cfg.intermediate),
            })
        self.final_norm = ones(E)
        self.lm_head = self.embed if cfg.tie_word_embeddings else rnd(cfg.vocab, E)
        self.inv_freq = 1.0 / (cfg.rope_theta ** (torch.arange(0, D, 2, dtype=torch.float32,
                                                               device=self.device) / D))
        shape = (cfg.num_layers, num_blocks, KV, block_size, D)
        self.fp8 = kv_cache_dtype == "fp8"
        if self.fp8:
            self.k_cache = torch.zeros(shape, dtype=torch.uint8,
                                       device=self.device).view(torch.float8_e4m3fn)
            self.v_cache = torch.zeros(shape, dtype=torch.uint8,
                                       device=self.device).view(torch.float8_e4m3fn)
            self.k_scale = torch.full((cfg.num_layers, KV), float(kv_scale), dtype=torch.float32,
                                      device=self.device)
            self.v_scale = self.k_scale.clone()
        else:
            self.k_cache = torch.zeros(shape, dtype=dtype, device=self.device)
            self.v_cache = torch.zeros(shape, dtype=dtype, device=self.device)

    # -- pieces ------------------------------------------------------------
    def _rope(self, x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor) -> torch.Tensor:
        """Rotate-half RoPE (HF Qwen3 apply_rotary_pos_emb), in fp32."""
        half = x.size(-1) // 2
        xf = x.float()
        x1, x2 = xf[..., :half], xf[..., half:]
        return torch.cat([x1 * cos - x2 * sin, x2 * cos + x1 * sin], dim=-1).to(x.dtype)

    def _rms_norm_heads(self, x: torch.Tensor, w: Optional[torch.Tensor]) -> torch.Tensor:
        """HF Qwen3RMSNorm over head_dim: fp32 statistics, round, times w
        (x itself for layers without q/k norms)."""
        if w is None:
            return x
        xf = x.float()
        r = torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + self.cfg.rms_eps)
        return w * (xf * r).to(x.dtype)

    def _prologue(self, li: int, w: dict, qkv: torch.Tensor, q: torch.Tensor, b: StepBatch,
                  rope) -> None:
        """q/k norm + RoPE into q, K/V of the step into layer li's pool."""
        cfg = self.cfg
        H, KV, D = cfg.num_heads, cfg.num_kv_heads, cfg.head_dim
        kc, vc = self.k_cache[li], self.v_cache[li]
        scales = (self.k_scale[li], self.v_scale[li]) if self.fp8 else (None, None)
        if self.fused_prologue:
            pk.qk_norm_rope_store(q, kc, vc, qkv, b.meta.slot_mapping, b.meta.positions,
                                  self.inv_freq, w["q_norm"], w["k_norm"], cfg.rms_eps, *scales)
            return
        T = qkv.size(0)
        cos, sin = rope
        qh = qkv[:, : H * D].view(T, H, D)
        k = qkv[:, H * D:(H + KV) * D].view(T, KV, D)
        v = qkv[:, (H + KV) * D:].view(T, KV, D)
        q.copy_(self._rope(self._rms_norm_heads(qh, w["q_norm"]), cos, sin))
        k = self._rope(self._rms_norm_heads(k, w["k_norm"]), cos, sin)
        if self.fp8:
            pk.paged_kv_store_slots_fp8(kc, vc, k, v, b.meta.slot_mapping, *scales)
        else:
            pk.paged_kv_store_slots(kc, vc, k, v, b.meta.slot_mapping)

    def _paged_attention(self, layer: int, q: torch.Tensor, kc: torch.Tensor, vc: torch.Tensor,
                         b: StepBatch, out: torch.Tensor) -> None:
        m, npf, tp = b.meta, b.num_prefill_seqs, b.num_prefill_tokens
        T = q.size(0)
        if npf:
            args = (out[:tp], q[:tp], kc, vc, m.block_tables[:npf], m.cu_seqlens_q[:npf + 1],
                    m.seq_lens[:npf], self.scale, self.block_size, m.max_blocks_per_seq,
                    max(1, b.max_prefill_q))
            if self.fp8:
                pk.paged_prefill_attention_fp8(*args, self.k_scale[layer], self.v_scale[layer],
                                               m.max_seq_len)
            else:
                pk.paged_prefill_attention(*args, m.max_seq_len)
        if T > tp:
            args = (out[tp:], q[tp:], kc, vc, m.block_tables[npf:], m.seq_lens[npf:], self.scale,
                    self.block_size, m.max_blocks_per_seq)
            if self.fp8:
                pk.paged_attention_forward_fp8(*args, self.k_scale[layer], self.v_scale[layer],
                                               workspace=b.decode_workspace)
            else:
                pk.paged_attention_forward(*args, workspace=b.decode_workspace)

    # -- forward -------------------------------------------------------------
    @torch.no_grad()
    def forward(self, b: StepBatch) -> torch.Tensor:
        """Runs one packed step; returns fp32 logits [R, vocab] of b.sample_rows
        (of every row when it is None)."""
        cfg = self.cfg
        H, KV, D, E = cfg.num_heads, cfg.num_kv_heads, cfg.head_dim, cfg.hidden
        T = b.input_ids.numel()
        rope = None
        if not self.fused_prologue:
            freqs = b.meta.positions.float()[:, None] * self.inv_freq[None, :]
            rope = (freqs.cos()[:, None, :], freqs.sin()[:, None, :])
        x = F.embedding(b.input_ids, self.embed)
        q = torch.empty(T, H, D, dtype=self.dtype, device=self.device)
        attn = torch.empty(T, H, D, dtype=self.dtype, device=self.device)
        for li, w in enumerate(self.layers):
            h = F.rms_norm(x, (E,), w["in_norm"], cfg.rms_eps)
            qkv = F.linear(h, w["qkv"], w["qkv_bias"])
            self._prologue(li, w, qkv, q, b, rope)
            kc, vc = self.k_cache[li], self.v_cache[li]
            self.attention(li, q, kc, vc, b, attn)
            x = x + attn.view(T, H * D) @ w["o"].t()
            h = F.rms_norm(x, (E,), w["post_norm"], cfg.rms_eps)
            gu = h @ w["gate_up"].t()
            x = x + (F.silu(gu[:, : cfg.intermediate]) * gu[:, cfg.intermediate:]) @ w["down"].t()
        if b.sample_rows is not None:
            x = x.index_select(0, b.sample_rows)
        xs = F.rms_norm(x, (E,), self.final_norm, cfg.rms_eps)
        return (xs @ self.lm_head.t()).float()

    @torch.no_grad()
    def load_hf_state_dict(self, sd: dict) -> None:
        """Takes the weights of a Hugging Face Qwen3ForCausalLM (or, with the
        Qwen2 options, Qwen2ForCausalLM) state dict (the models the reference's
        ModelRunner wraps, nanoPD/engine/model_runner.py:8-13, :53-58): q/k/v
        projections fused into one [(H + 2 KV) * D, E] matrix (and their
        biases into one vector), gate/up into one [2 I, E], the rest as they
        are. An untied model needs lm_head.weight; a tied one shares the
        embedding."""
        def get(name):
            t = sd[name]
            return t.to(device=self.device, dtype=self.dtype)

        self.embed.copy_(get("model.embed_tokens.weight"))
        for i, w in enumerate(self.layers):
            p = f"model.layers.{i}."
            w["in_norm"].copy_(get(p + "input_layernorm.weight"))
            w["qkv"].copy_(torch.cat([get(p + "self_attn.q_proj.weight"),
                                      get(p + "self_attn.k_proj.weight"),
                                      get(p + "self_attn.v_proj.weight")], dim=0))
            if self.cfg.qkv_bias:
                w["qkv_bias"].copy_(torch.cat([get(p + "self_attn.q_proj.bias"),
                                               get(p + "self_attn.k_proj.bias"),
                                               get(p + "self_attn.v_proj.bias")], dim=0))
            if self.cfg.qk_norm:
                w["q_norm"].copy_(get(p + "self_attn.q_norm.weight"))
                w["k_norm"].copy_(get(p + "self_attn.k_norm.weight"))
            w["o"].copy_(get(p + "self_attn.o_proj.weight"))
            w["post_norm"].copy_(get(p + "post_attention_layernorm.weight"))
            w["gate_up"].copy_(torch.cat([get(p + "mlp.gate_proj.weight"),
                                          get(p + "mlp.up_proj.weight")], dim=0))
            w["down"].copy_(get(p + "mlp.down_proj.weight"))
        self.final_norm.copy_(get("model.norm.weight"))
        if not self.cfg.tie_word_embeddings:   # an untied head without its own weight: the embedding
            self.lm_head.copy_(get("lm_head.weight" if "lm_head.weight" in sd
                                   else "model.embed_tokens.weight"))

    def copy_blocks(self, pairs) -> None:
        """Copy-on-write copies (old, new) in every layer's cache."""
        if not pairs:
            return
        t = torch.tensor(pairs, dtype=torch.int32).to(self.device)
        for li in range(self.cfg.num_layers):
            pk.copy_blocks(self.k_cache[li], self.v_cache[li], t)
