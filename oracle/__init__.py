"""CPU oracle for the TuringServe per-step hot path -- TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py`` may
import this package, and only as the checker; the product (``turingserve_amd``) never does.

Contents (numpy; every function cites the reference file:line it restates):

* ``oracle.paged``  -- kv_write scatter, slot mapping, block-table gather, the masked attention
  of ``ops/reference.py:60-77``, ``paged_attention`` of ``ops/reference.py:94-111``, the split-K
  merge of ``ops/triton_decode_attention.py:144-163`` and a pure-Python brute force.
* ``oracle.quant``  -- per-row int8 quantisation ``quant/int8.py:8-16`` and the W8A16 product
  ``ops/triton_w8a16.py:11-35`` / the twin ``ops/reference.py:45-47``.

How each function is pinned (the reference stores no golden vectors for this path): see the
tests in ``tests/test_oracle.py`` -- fp64 brute-force loops, closed forms (identity weights,
scale = 1 integer products), the split-K merge against a single pass, paged == contiguous, needle
constructions and the quantisation error bound. No function here is left unpinned.
"""
