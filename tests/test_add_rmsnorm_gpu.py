"""The W8A16 product fused with the residual add and RMSNorm that consume it
(ts_w8a16_add_rmsnorm; model/qwen2.py:84-92's rmsnorm_residual(linear(x, proj), residual)) on the
GPU.

It must equal, bit for bit, the pair it replaces -- ts_w8a16_gemm_v with the same variant and
splits, then ts_rmsnorm with the residual -- on every path the plan takes (skinny, weight
streaming, the wide tiles, split-K, where the norm launch reduces the partials itself), with
bias and fp16 scales; both halves of that pair are pinned to their oracles by the GEMM and
small-op tests. The model's forward (which takes every o_proj and down_proj this way) must equal
the unfused layer-by-layer chain.
"""

from __future__ import annotations

import pytest
import torch

from oracle import quant as OQ
from turingserve_amd import hip_ops as K

pytestmark = pytest.mark.gpu
DEV = "cuda"
EPS = 1e-6


def _problem(M, Nn, Kd, seed, bias=False, fp16_scale=False):
    g = torch.Generator().manual_seed(seed)
    w = torch.randn(Nn, Kd, generator=g) * 0.05
    wq, sc = OQ.quantize(w.numpy())
    x = torch.randn(M, Kd, generator=g).half()
    res = (torch.randn(M, Nn, generator=g) * 2).half()
    nw = (1 + 0.1 * torch.randn(Nn, generator=g)).half()
    b = (torch.randn(Nn, generator=g) * 0.1).half() if bias else None
    scale = torch.from_numpy(sc)
    if fp16_scale:
        scale = scale.half()
    return (x.to(DEV), torch.from_numpy(wq).to(DEV), scale.to(DEV),
            None if b is None else b.to(DEV), res.to(DEV), nw.to(DEV))


def _unfused(x, wq, scale, b, res, nw, cfg):
    return K.rmsnorm_residual(K.w8a16_linear(x, wq, scale, b, cfg), res, nw, EPS)


@pytest.mark.parametrize("M,Nn,Kd", [
    (1, 1536, 1536), (16, 1536, 1536), (64, 1536, 1536), (560, 1536, 1536),   # 1.5B o_proj
    (1, 1536, 8960), (64, 1536, 8960), (560, 1536, 8960), (2048, 1536, 8960),  # 1.5B down_proj
    (7, 896, 4864), (33, 64, 200)])
def test_add_rmsnorm_equals_gemm_then_norm(M, Nn, Kd):
    x, wq, scale, _, res, nw = _problem(M, Nn, Kd, seed=M + Nn + Kd)
    out, res_out = K.w8a16_add_rmsnorm(x, wq, scale, None, res, nw, EPS)
    want_out, want_res = _unfused(x, wq, scale, None, res, nw, None)
    assert torch.equal(res_out, want_res) and torch.equal(out, want_out)


@pytest.mark.parametrize("variant,splits", [(1, 0), (1, 3), (2, 0), (2, 4), (3, 0), (4, 2),
                                            (4, 8), (5, 0), (6, 0), (7, 0)])
@pytest.mark.parametrize("M", [2, 9, 64, 200])
def test_add_rmsnorm_every_variant_and_split(variant, splits, M):
    if variant == 7 and M > 4:
        pytest.skip("the VALU path is built for M <= 4")
    if variant == 1 and M > 32:
        pytest.skip("weight streaming is built for M <= 32")
    if variant == 5 and M > 64:
        pytest.skip("the skinny kernel is built for M <= 64")
    x, wq, scale, b, res, nw = _problem(M, 1024, 1536, seed=variant * 10 + splits + M, bias=True,
                                        fp16_scale=True)
    cfg = (variant, splits)
    out, res_out = K.w8a16_add_rmsnorm(x, wq, scale, b, res, nw, EPS, cfg)
    want_out, want_res = _unfused(x, wq, scale, b, res, nw, cfg)
    assert torch.equal(res_out, want_res) and torch.equal(out, want_out)


def test_add_rmsnorm_empty_and_routing():
    from turingserve_amd import get_ops
    from turingserve_amd.qwen2 import TINY_G2, random_weights

    x, wq, scale, _, res, nw = _problem(3, 64, 64, seed=1)
    out, res_out = K.w8a16_add_rmsnorm(x[:0], wq, scale, None, res[:0], nw, EPS)
    assert out.shape == res_out.shape == (0, 64)
    ops = get_ops("hip")
    h = torch.randn(11, TINY_G2.hidden_size, device=DEV).half()
    r = torch.randn(11, TINY_G2.hidden_size, device=DEV).half()
    for quantization in ("int8", "none"):                 # fused call / the two calls
        lw = random_weights(TINY_G2, DEV, seed=4, quantization=quantization).layers[0]
        got = ops.linear_rmsnorm_residual(h, lw.o_proj, r, lw.post_attention_norm, EPS)
        want = ops.rmsnorm_residual(ops.linear(h, lw.o_proj), r, lw.post_attention_norm, EPS)
        assert torch.equal(got[0], want[0]) and torch.equal(got[1], want[1])


@pytest.mark.parametrize("cfg_name", ["TINY_G2", "D128"])
def test_forward_equals_layer_chain(cfg_name):
    """Qwen2Model.forward (each down_proj fused into the next norm, each o_proj into
    post_attention_layernorm) against layer_forward over every layer and the final norm."""
    from turingserve_amd import get_ops
    from turingserve_amd.metadata import BatchItem, InputBuilder, SeqState
    from turingserve_amd.qwen2 import TINY_G2, Qwen2Config, Qwen2Model, random_weights

    cfg = TINY_G2 if cfg_name == "TINY_G2" else Qwen2Config(768, 1536, 2, 6, 1, 4096,
                                                            max_position_embeddings=4096)
    model = Qwen2Model(cfg, random_weights(cfg, DEV, seed=2, quantization="int8"), get_ops("hip"),
                       max_model_len=4096)
    ids = [(7 * i + 3) % cfg.vocab_size for i in range(300)]
    items = [BatchItem(SeqState(ids, list(range(1, 20))), 0, ids, "all")]
    inp = InputBuilder(512, 4, 64, DEV).build(items)
    with torch.inference_mode():
        kv1, kv2 = model.new_kv_cache(64), model.new_kv_cache(64)
        got = model.forward(inp.input_ids, inp.positions, inp.meta, kv1)
        h, res = model.w.embed_tokens[inp.input_ids], None
        for i in range(len(model.w.layers)):
            h, res = model.layer_forward(i, h, res, inp.positions, inp.meta, kv2)
        want = model.ops.rmsnorm_residual(h, res, model.w.final_norm, cfg.rms_norm_eps)[0]
    assert torch.equal(got, want) and torch.equal(kv1, kv2)
