"""Qwen2 forward over a flat ragged token batch, through an op namespace.

The caller of the hot path (model/qwen2.py:24-99): per layer rmsnorm(+residual) -> fused qkv
linear -> in-place RoPE -> kv_write of the new K/V rows -> paged attention -> o linear ->
rmsnorm(+residual) -> fused gate_up linear -> silu * up -> down linear; a final norm and the tied
embedding as lm head for the sampling rows only. Weights are random (seeded) because no checkpoint
is available offline; the fused layouts match the loader's (model/loader.py:68-92): qkv =
[q; k; v] with bias, gate_up = [gate; up], optional per-row int8 (W8A16) linears.
"""

from __future__ import annotations

from dataclasses import dataclass

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


def rope_tables(head_dim: int, theta: float, max_len: int, device) -> tuple[torch.Tensor, torch.Tensor]:
    """(cos, sin) [max_len, D/2] fp32 for rotate-half RoPE. The inverse frequencies are formed
    exactly as Hugging Face's Qwen2 rotary embedding forms them, so the tables hold the same
    bits as a checkpoint's own inference would use (model/layers.py:10-18 does the same)."""
    exponent = torch.arange(0, head_dim, 2, dtype=torch.int64).float() / head_dim
    angle = torch.outer(torch.arange(max_len).float(), 1.0 / (theta ** exponent))
    return angle.cos().to(device), angle.sin().to(device)


@dataclass
class DecoderLayer:
    """One decoder layer's parameters in the fused layouts the ops take (model/loader.py:82-92):
    qkv_proj = [q; k; v] rows with a bias, gate_up_proj = [gate; up] rows."""

    input_norm: torch.Tensor
    qkv_proj: LinearWeight
    o_proj: LinearWeight
    post_attention_norm: torch.Tensor
    gate_up_proj: LinearWeight
    down_proj: LinearWeight


@dataclass
class Qwen2Weights:
    """The model's parameters. embed_tokens [V, hidden] is also the (tied) lm head;
    lm_head_int8 = (int8 [V, hidden], scale [V]) when the lm head runs as W8A16."""

    embed_tokens: torch.Tensor
    layers: list[DecoderLayer]
    final_norm: torch.Tensor
    lm_head_int8: tuple[torch.Tensor, torch.Tensor] | None = None


def random_weights(cfg: Qwen2Config, device, dtype=torch.float16, seed: int = 0,
                   quantization: str = "none", init_std: float = 0.2,
                   int8_lm_head: bool = False, draw_on: str = "device") -> Qwen2Weights:
    """Seeded random weights in the loader's fused layouts. draw_on="device" draws with a
    generator on `device` when it is a GPU (the 1.5B shapes initialise in seconds); "cpu" draws on
    the host and moves the result, so the same seed gives the same weights on any device (the
    end-to-end tests pick their seeds on the CPU). init_std 0.2 is the tiny models'
    initializer_range; the 1.5B configuration uses a smaller std so activations stay in fp16
    range. Norm weights are 1 + N(0, 0.1)."""
    gpu_draw = draw_on == "device" and torch.device(device).type == "cuda"
    where = device if gpu_draw else "cpu"
    g = torch.Generator(device=where).manual_seed(seed)

    def normal(*shape, std=init_std):
        return torch.randn(*shape, generator=g, device=where) * std

    def norm_weight(n):
        return (1.0 + normal(n, std=0.1)).to(dtype).to(device)

    def proj(n, k, bias=False):
        w = normal(n, k).to(dtype)
        b = normal(n).to(dtype).to(device) if bias else None
        if quantization == "int8":
            wq, scale = quantize(w.float())
            return LinearWeight(wq.to(device), b, scale.to(device))
        return LinearWeight(w.to(device), b)

    hid, D, inter = cfg.hidden_size, cfg.head_dim, cfg.intermediate_size
    layers = [DecoderLayer(input_norm=norm_weight(hid),
                           qkv_proj=proj(cfg.qkv_dim, hid, bias=True),
                           o_proj=proj(hid, cfg.num_heads * D),
                           post_attention_norm=norm_weight(hid),
                           gate_up_proj=proj(2 * inter, hid),
                           down_proj=proj(hid, inter))
              for _ in range(cfg.num_layers)]
    embed = normal(cfg.vocab_size, hid).to(dtype).to(device)
    head = None
    if int8_lm_head:
        wq, scale = quantize(embed.float())
        head = (wq.to(device), scale.to(device))
    return Qwen2Weights(embed, layers, norm_weight(hid), head)


class Qwen2Model:
    """The forward pass over one flat ragged batch; `ops` is a get_ops() namespace. Device and
    activation dtype are the embedding's."""

    def __init__(self, cfg: Qwen2Config, weights: Qwen2Weights, ops,
                 max_model_len: int | None = None) -> None:
        self.cfg, self.w, self.ops = cfg, weights, ops
        self.device = weights.embed_tokens.device
        self.dtype = weights.embed_tokens.dtype
        self.scale = cfg.head_dim ** -0.5
        self.cos, self.sin = rope_tables(cfg.head_dim, cfg.rope_theta,
                                         max_model_len or cfg.max_position_embeddings,
                                         self.device)

    def _rotate_write(self, qkv, positions, k_cache, v_cache, slot_mapping):
        c = self.cfg
        fused = getattr(self.ops, "rope_kv_write_", None)
        args = (qkv, positions, self.cos, self.sin, c.num_heads, c.num_kv_heads,
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

    def _mlp_act(self, x, lw):
        """silu(gate) * up, the input of down_proj."""
        gate_up_silu = getattr(self.ops, "gate_up_silu", None)       # fused on the hip backend
        return (gate_up_silu(x, lw.gate_up_proj) if gate_up_silu is not None
                else self.ops.silu_mul(self.ops.linear(x, lw.gate_up_proj)))

    def _project_norm(self, x, proj, residual, norm_w):
        """rmsnorm_residual(linear(x, proj), residual, norm_w): on a backend that has
        linear_rmsnorm_residual the product's split-K reduction runs inside the norm launch
        (same values as the two calls)."""
        fused = getattr(self.ops, "linear_rmsnorm_residual", None)
        if fused is not None:
            return fused(x, proj, residual, norm_w, self.cfg.rms_norm_eps)
        return self.ops.rmsnorm_residual(self.ops.linear(x, proj), residual, norm_w,
                                         self.cfg.rms_norm_eps)

    def pure_decode(self, meta, num_tokens: int) -> bool:
        """True when every row of the step is a decode row (the fused decode launch applies)."""
        return meta.num_decode == num_tokens and meta.seq_lens.shape[0] == meta.num_decode

    def _attention_block(self, index: int, x, residual, positions, meta, kv_cache,
                         fused_decode: bool, split_map=None):
        """Decoder layer `index` from its normed input x to the MLP activation: qkv, RoPE, the
        K/V write into kv_cache[index], attention, o_proj with post_attention_layernorm, and
        silu(gate) * up; returns (the input of down_proj, residual). split_map: the step's
        decode split map (fused decode only), shared by every layer."""
        c, ops, lw = self.cfg, self.ops, self.w.layers[index]
        k_cache, v_cache = kv_cache[index, 0], kv_cache[index, 1]
        H, KVH, D = c.num_heads, c.num_kv_heads, c.head_dim
        a = None
        qkv_rope = getattr(ops, "linear_rope_kv_write", None)
        if fused_decode and hasattr(ops, "decode_rope_kv_write_attention"):
            qkv = ops.linear(x, lw.qkv_proj)
            a = ops.decode_rope_kv_write_attention(qkv, positions, self.cos, self.sin, H, KVH, D,
                                                   k_cache, v_cache, meta, self.scale,
                                                   split_map=split_map)
            if a is None:             # a layout the fused launch does not take
                q, _, _ = self._rotate_write(qkv, positions, k_cache, v_cache, meta.slot_mapping)
        elif qkv_rope is not None:    # the product, RoPE and the cache write in one call
            qkv = qkv_rope(x, lw.qkv_proj, positions, self.cos, self.sin, H, KVH, D, k_cache,
                           v_cache, meta.slot_mapping)
            q = qkv[:, :H * D].view(qkv.shape[0], H, D)
        else:
            q, _, _ = self._rotate_write(ops.linear(x, lw.qkv_proj), positions, k_cache, v_cache,
                                         meta.slot_mapping)
        if a is None:
            a = ops.paged_attention(q, k_cache, v_cache, meta, self.scale)
        x, residual = self._project_norm(a, lw.o_proj, residual, lw.post_attention_norm)
        return self._mlp_act(x, lw), residual

    @torch.inference_mode()
    def layer_forward(self, index: int, h, residual, positions, meta, kv_cache,
                      fused_decode: bool = False):
        """Decoder layer `index` (model/qwen2.py:84-92): (h, residual) in, (h, residual) out,
        residual None before the first layer. The layer's new K/V rows go into kv_cache[index]
        before its attention reads it. With fused_decode (a pure-decode step on a backend that
        has decode_rope_kv_write_attention), RoPE, kv_write and attention run as one launch
        (same outputs and caches as the three calls)."""
        c, lw = self.cfg, self.w.layers[index]
        if residual is None:
            residual = h
            x = self.ops.rmsnorm(h, lw.input_norm, c.rms_norm_eps)
        else:
            x, residual = self.ops.rmsnorm_residual(h, residual, lw.input_norm, c.rms_norm_eps)
        act, residual = self._attention_block(index, x, residual, positions, meta, kv_cache,
                                              fused_decode)
        return self.ops.linear(act, lw.down_proj), residual

    @torch.inference_mode()
    def forward(self, input_ids, positions, meta, kv_cache):
        """kv_cache [L, 2, num_blocks, KVH, 16, D] -> final normed hidden rows [T, hidden].
        The same chain as layer_forward over every layer and the final norm, with each layer's
        down_proj taken together with the norm that consumes it (the next input_layernorm, or
        the final norm): the same values, without a separate split-K reduction launch."""
        c, layers = self.cfg, self.w.layers
        fused = self.pure_decode(meta, input_ids.shape[0])
        # one decode split map per step, read by every layer's fused decode launch
        build_map = getattr(self.ops, "decode_split_map", None) if fused else None
        split_map = (build_map(meta, c.num_heads, c.num_kv_heads, c.head_dim, kv_cache.shape[2],
                               kv_cache.device) if build_map is not None else None)
        h = self.w.embed_tokens[input_ids]
        residual = h
        x = self.ops.rmsnorm(h, layers[0].input_norm, c.rms_norm_eps)
        for index in range(len(layers)):
            act, residual = self._attention_block(index, x, residual, positions, meta, kv_cache,
                                                  fused, split_map)
            norm_w = layers[index + 1].input_norm if index + 1 < len(layers) else self.w.final_norm
            x, residual = self._project_norm(act, layers[index].down_proj, residual, norm_w)
        return x

    def compute_logits(self, hidden: torch.Tensor, sample_indices: torch.Tensor) -> torch.Tensor:
        """Logits of the sampling rows only, [S, V] fp32 (model/qwen2.py:94-99). With the int8
        lm head, a backend that has logits_int8 gathers, multiplies and widens in one launch
        (same values as lm_head_int8 on the gathered rows followed by .float())."""
        head = self.w.lm_head_int8
        if head is not None and hasattr(self.ops, "logits_int8"):
            return self.ops.logits_int8(hidden, sample_indices, *head)
        h = hidden[sample_indices]
        if head is not None and hasattr(self.ops, "lm_head_int8"):
            return self.ops.lm_head_int8(h, *head).float()
        return (h @ self.w.embed_tokens.T).float()

    def new_kv_cache(self, num_blocks: int) -> torch.Tensor:
        c = self.cfg
        return torch.zeros(c.num_layers, 2, num_blocks, c.num_kv_heads, 16, c.head_dim,
                           dtype=self.dtype, device=self.device)
