"""Op dispatch: ``get_ops("reference" | "hip")`` returns a namespace of op callables.

Restates ops/__init__.py:12-43 with ``hip`` in place of ``triton``: the hip namespace starts from
the reference namespace (the dense/masked attention helpers stay on the twins) and overrides the
hot-path ops and the fused small ops with the gfx950 kernels. ``"triton"`` is accepted as an alias
of ``"hip"`` so an existing ``--kernels triton`` configuration switches backends unchanged.
"""

from __future__ import annotations

from types import SimpleNamespace


def _reference() -> SimpleNamespace:
    from turingserve_amd import reference_ops as r

    return SimpleNamespace(
        name="reference", rmsnorm=r.rmsnorm, rmsnorm_residual=r.rmsnorm_residual,
        silu_mul=r.silu_mul, rope_=r.rope_, linear=r.linear, kv_write=r.kv_write,
        paged_attention=r.paged_attention, dense_causal_attention=r.dense_causal_attention,
        attention_with_mask=r.attention_with_mask)


def _hip() -> SimpleNamespace:
    from turingserve_amd import _native
    from turingserve_amd import hip_ops as h

    _native.lib()                 # fail now, loudly, if the kernel library is missing
    ns = _reference()
    ns.name = "hip"
    ns.linear = h.linear
    ns.kv_write = h.kv_write
    ns.paged_attention = h.paged_attention
    ns.lm_head_int8 = h.lm_head_int8
    ns.logits_int8 = h.logits_int8
    ns.rmsnorm = h.rmsnorm
    ns.rmsnorm_residual = h.rmsnorm_residual
    ns.rope_ = h.rope_
    ns.silu_mul = h.silu_mul
    ns.gate_up_silu = h.gate_up_silu
    ns.linear_rmsnorm_residual = h.linear_rmsnorm_residual
    ns.rope_kv_write_ = h.rope_kv_write_
    ns.decode_rope_kv_write_attention = h.decode_rope_kv_write_attention
    ns.decode_split_map = h.decode_split_map
    ns.linear_rope_kv_write = h.linear_rope_kv_write
    return ns


def get_ops(kernels: str) -> SimpleNamespace:
    if kernels == "reference":
        return _reference()
    if kernels in ("hip", "triton"):
        return _hip()
    raise ValueError(f"unknown kernels backend {kernels!r}")
