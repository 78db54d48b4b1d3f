"""CPU oracle for the DSA decoder-layer hot path (test infrastructure only).

This package restates, on the CPU, the arithmetic of the reference monokernel
(``sgl_amd_mono/glm53/gfx950/kernel.py`` and the DeepSeek-V4 indexer stages) for one
GPU's TP=4 share of a DeepSeek-V3.2-geometry decoder layer. It is the checker the
parity tests, ``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline`` leg
compare the HIP kernels against. Nothing in the product path imports it.

Modules:

* ``formats``  number formats: E4M3, E8M0, E2M1, per-128 FP8 activation quant,
  the radix order key.
* ``front``    RMSNorm, LayerNorm, RoPE, FWHT-128, the FP4 and FP8 quantisers, and the
  front of the layer: projections, KV row, index key and query chains, absorbed query.
* ``attn``     the FP4 indexer scores, the chain's exact top-k, sparse MLA decode.
* ``dense``    the W8A16 block-scaled GEMV and the output block (W_UV, o_proj, residual).
* ``moe``      RMSNorm, router, sigmoid top-8 routing, FP8 W8A8 and MXFP4 A16W4
  expert SwiGLU, the bf16 softmax top-2 plumbing block.
* ``topk``     the exact top-k selection: a sort-based restatement and the radix
  select in plain C (``topk.c``, built into ``liboracle_topk.so`` by ``oracle/Makefile``)
  used at full sizes.

Every function cites the reference file:line it follows. How each is pinned (by a
library routine, a closed form, brute force, or the reference's test formulas) is
recorded in its docstring under "Pinned by"; a function with no such check says
"parity unpinned".
"""
