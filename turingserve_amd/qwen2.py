"""Qwen2 forward over a flat ragged token batch, through an op namespace.

The caller of the hot path (model/qwen2.py:24-99): per layer rmsnorm(+residual) -> fused qkv
linear -> in-place RoPE -> kv_write of the new K/V rows -> paged attention -> o linear ->
rmsnorm(+residual) -> fused gate_up linear -> silu * up -> down linear; a final norm and the tied
embedding as lm head for the sampling rows only. Weights are random (seeded) because no checkpoint
is available offline; the fused layouts match the loader's (model/loader.py:68-92): qkv =
[q; k; v] with bias, gate_up = [gate; up], optional per-row int8 (W8A16) linears.
"""

from __future__ import annotations

from dataclasses import dataclass, field

import torch

from turingserve_amd.quant import LinearWeight, quantize


@dataclass(frozen=True)
class Qwen2Config:
    hidden_size: int
    intermediate_size: int
    num_layers: int
    num_heads: int
    num_kv_heads: int
    vocab_size: int
    rms_norm_eps: float = 1e-6
    rope_theta: float = 1e6
    max_position_embeddings: int = 32768

    @property
    def head_dim(self) -> int:
        return self.hidden_size // self.num_heads

    @property
    def qkv_dim(self) -> int:
        return (self.num_heads + 2 * self.num_kv_heads) * self.head_dim

    @property
    def kv_bytes_per_token(self) -> int:
        """K and V x layers x KVH x D x 2 bytes (model/qwen2_config.py:31-34)."""
        return 2 * self.num_layers * self.num_kv_heads * self.head_dim * 2


# The tiny test models of the reference (scripts/make_tiny_model.py:27-31) and Qwen2.5-1.5B.
TINY_G2 = Qwen2Config(64, 128, 2, 4, 2, 151936, max_position_embeddings=4096)
TINY_G7 = Qwen2Config(224, 448, 2, 14, 2, 151936, max_position_embeddings=4096)
QWEN25_15B = Qwen2Config(1536, 8960, 28, 12, 2, 151936)


class RotaryCache:
    """cos / sin tables [max_len, D/2] in fp32, cast to the activation dtype at use
    (model/layers.py:10-18)."""

    def __init__(self, head_dim: int, theta: float, max_len: int, device) -> None:
        inv_freq = 1.0 / (theta ** (torch.arange(0, head_dim, 2, dtype=torch.int64).float() / head_dim))
        freqs = torch.outer(torch.arange(max_len).float(), inv_freq)
        self.cos = freqs.cos().to(device)
        self.sin = freqs.sin().to(device)


@dataclass
class LayerWeights:
    w_in: torch.Tensor
    qkv: LinearWeight
    o: LinearWeight
    w_post: torch.Tensor
    gu: LinearWeight
    down: LinearWeight


@dataclass
class Weights:
    embed: torch.Tensor                       # [V, hidden], also the tied lm head
    layers: list[LayerWeights] = field(default_factory=list)
    w_norm: torch.Tensor | None = None
    embed_q: tuple[torch.Tensor, torch.Tensor] | None = None   # optional int8 lm head


def random_weights(cfg: Qwen2Config, device, dtype=torch.float16, seed: int = 0,
                   quantization: str = "none", init_std: float = 0.2,
                   int8_lm_head: bool = False) -> Weights:
    """Seeded random weights with the loader's fused layouts, drawn on `device` (a GPU generator
    when it is one, so the 1.5B shapes initialise in seconds). init_std 0.2 (the tiny models'
    initializer_range) spreads the logits so greedy ties are rare; the large configuration uses a
    smaller std so activations stay in fp16 range."""
    on_device = torch.device(device).type == "cuda"
    g = torch.Generator(device=device if on_device else "cpu").manual_seed(seed)
    gen_dev = device if on_device else "cpu"

    def rnd(*shape, std=init_std):
        return torch.randn(*shape, generator=g, device=gen_dev) * std

    def lin(n, k, bias=False):
        w = rnd(n, k).to(dtype)
        b = rnd(n).to(dtype).to(device) if bias else None
        if quantization == "int8":
            wq, scale = quantize(w.float())
            return LinearWeight(wq.to(device), b, scale.to(device))
        return LinearWeight(w.to(device), b)

    H, D, I = cfg.hidden_size, cfg.head_dim, cfg.intermediate_size
    layers = []
    for _ in range(cfg.num_layers):
        layers.append(LayerWeights(
            w_in=(1.0 + 0.1 * rnd(H, std=1.0)).to(dtype).to(device),
            qkv=lin(cfg.qkv_dim, H, bias=True),
            o=lin(H, cfg.num_heads * D),
            w_post=(1.0 + 0.1 * rnd(H, std=1.0)).to(dtype).to(device),
            gu=lin(2 * I, H),
            down=lin(H, I)))
    embed = rnd(cfg.vocab_size, H).to(dtype).to(device)
    w = Weights(embed=embed, layers=layers,
                w_norm=(1.0 + 0.1 * rnd(H, std=1.0)).to(dtype).to(device))
    if int8_lm_head:
        wq, scale = quantize(embed.float())
        w.embed_q = (wq, scale)
    return w


class Qwen2Model:
    def __init__(self, cfg: Qwen2Config, weights: Weights, ops, device,
                 dtype: torch.dtype = torch.float16, max_model_len: int | None = None) -> None:
        self.cfg = cfg
        self.w = weights
        self.ops = ops
        self.device = device
        self.dtype = dtype
        self.scale = cfg.head_dim ** -0.5
        self.rotary = RotaryCache(cfg.head_dim, cfg.rope_theta,
                                  max_model_len or cfg.max_position_embeddings, device)

    def _qkv(self, x, lw, positions, k_cache, v_cache, slot_mapping):
        """q, k, v views of the rotated qkv activation, with the new K / V rows already in the
        layer's cache (model/qwen2.py:26-28 and :89: rope, then kv_write). A backend with
        rope_kv_write_ rotates and writes them in one pass."""
        return self._rotate_write(self.ops.linear(x, lw.qkv), positions, k_cache, v_cache,
                                  slot_mapping)

    def _rotate_write(self, qkv, positions, k_cache, v_cache, slot_mapping):
        c = self.cfg
        fused = getattr(self.ops, "rope_kv_write_", None)
        args = (qkv, positions, self.rotary.cos, self.rotary.sin, c.num_heads, c.num_kv_heads,
                c.head_dim)
        written = fused is not None and fused(*args, k_cache, v_cache, slot_mapping)
        if not written:
            self.ops.rope_(*args)
        T, H, KVH, D = qkv.shape[0], c.num_heads, c.num_kv_heads, c.head_dim
        q = qkv[:, : H * D].view(T, H, D)
        k = qkv[:, H * D:(H + KVH) * D].view(T, KVH, D)
        v = qkv[:, (H + KVH) * D:].view(T, KVH, D)
        if not written:
            self.ops.kv_write(k, v, k_cache, v_cache, slot_mapping)
        return q, k, v

    def _mlp(self, x, lw):
        gate_up_silu = getattr(self.ops, "gate_up_silu", None)       # fused on the hip backend
        act = (gate_up_silu(x, lw.gu) if gate_up_silu is not None
               else self.ops.silu_mul(self.ops.linear(x, lw.gu)))
        return self.ops.linear(act, lw.down)

    @torch.inference_mode()
    def forward(self, input_ids, positions, meta, kv_cache):
        """kv_cache [L, 2, num_blocks, KVH, 16, D]; per layer kv_write first, then attention
        (model/qwen2.py:84-92)."""
        c, ops, w = self.cfg, self.ops, self.w
        h = w.embed[input_ids]
        residual = None
        # A pure-decode step on a backend that fuses rope, kv_write and decode attention into one
        # launch takes that path (same outputs and caches as the three calls).
        fused_decode = getattr(ops, "decode_rope_kv_write_attention", None)
        if fused_decode is not None and not (meta.num_decode == input_ids.shape[0]
                                             and meta.seq_lens.shape[0] == meta.num_decode):
            fused_decode = None
        for layer, lw in enumerate(w.layers):
            if residual is None:
                residual = h
                x = ops.rmsnorm(h, lw.w_in, c.rms_norm_eps)
            else:
                x, residual = ops.rmsnorm_residual(h, residual, lw.w_in, c.rms_norm_eps)
            k_cache, v_cache = kv_cache[layer, 0], kv_cache[layer, 1]
            a = None
            if fused_decode is not None:
                qkv = ops.linear(x, lw.qkv)
                a = fused_decode(qkv, positions, self.rotary.cos, self.rotary.sin, c.num_heads,
                                 c.num_kv_heads, c.head_dim, k_cache, v_cache, meta, self.scale)
                if a is None:                   # layout the fused launch does not take
                    fused_decode = None
                    q, _, _ = self._rotate_write(qkv, positions, k_cache, v_cache,
                                                 meta.slot_mapping)
                    a = ops.paged_attention(q, k_cache, v_cache, meta, self.scale)
            if a is None:
                q, _, _ = self._qkv(x, lw, positions, k_cache, v_cache, meta.slot_mapping)
                a = ops.paged_attention(q, k_cache, v_cache, meta, self.scale)
            h = ops.linear(a, lw.o)
            x, residual = ops.rmsnorm_residual(h, residual, lw.w_post, c.rms_norm_eps)
            h = self._mlp(x, lw)
        x, _ = ops.rmsnorm_residual(h, residual, w.w_norm, c.rms_norm_eps)
        return x

    def compute_logits(self, hidden: torch.Tensor, sample_indices: torch.Tensor) -> torch.Tensor:
        """Logits of the sampling rows only, [S, V] fp32 (model/qwen2.py:94-99). With the int8
        lm head, a backend that has logits_int8 gathers, multiplies and widens in one launch
        (same values as lm_head_int8 on the gathered rows followed by .float())."""
        if self.w.embed_q is not None and hasattr(self.ops, "logits_int8"):
            return self.ops.logits_int8(hidden, sample_indices, *self.w.embed_q)
        h = hidden[sample_indices]
        if self.w.embed_q is not None and hasattr(self.ops, "lm_head_int8"):
            return self.ops.lm_head_int8(h, *self.w.embed_q).float()
        return (h @ self.w.embed.T).float()

    def new_kv_cache(self, num_blocks: int) -> torch.Tensor:
        c = self.cfg
        return torch.zeros(c.num_layers, 2, num_blocks, c.num_kv_heads, 16, c.head_dim,
                           dtype=self.dtype, device=self.device)
