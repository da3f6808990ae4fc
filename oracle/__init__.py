"""CPU oracle for the Quest sparse-decode path (TEST INFRASTRUCTURE ONLY).

This package is a plain-numpy restatement of the reference algorithm
(wengyinqi/QwenQuest, ``src/qwenquest/quest.py``,
``src/qwenquest/hisparse/coordinator.py``, ``src/qwenquest/attention/ops.py``).
Every function cites the reference ``file:line`` it follows.

It exists only to *check* the HIP implementation.  Only ``tests/``,
``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py`` may
import it; the product package ``qwenquest_amd`` never does, and it has no CPU
fallback of its own.

Canonicalisations the oracle fixes (the reference leaves them to torch
internals, which differ between CPU ISAs and versions):

* ``page_scores`` - fp32 products (no fused multiply-add), summed per page in a
  fixed order: 64 lanes, lane ``l`` adds channels ``[l*m, (l+1)*m)`` in order
  (``m = ceil(KV*D / 64)``), then a halving tree over the 64 lane sums
  (``acc[i] += acc[i + w]`` for ``w = 32, 16, ..., 1``).
* top-k - descending score, ties broken by the LOWEST page index (torch.topk's
  tie order is implementation-defined).
* GQA mean - fp32 sum over the group in head order, divided by the group size,
  rounded once (RNE) to the query dtype.

Parity status per function (what pins it) is listed in ``PINNING`` below and
checked by ``tests/test_oracle_*.py``.
"""

PINNING = {
    "bf16 conversions": "closed form; round-trip and RNE tie cases vs torch",
    "init_storage / sentinels": "reference test known answers (test_quest_algorithm.py:62-69)",
    "prefill_bounds": "closed form min/max; reference known answers (test_quest_algorithm.py:72-98)",
    "decode_fold / finalize": "brute force vs prefill of the same tokens; known answers (:109-137)",
    "step_layout": "closed-form integer arithmetic; known answers (:170-183, :253-285)",
    "group_queries": "textbook mean; reference known answer (:227-234); torch bf16 mean on bf16 input",
    "page_scores": "exact products; naive loop (:211-224); upper-bound invariant (:198-208); "
    "reference golden vectors within fp32 ulps (tests/golden)",
    "topk_pages": "stable sort of (-score, page); planted page (:186-192); golden vectors",
    "decode_attention": "float64 textbook softmax attention; torch SDPA on expanded rows",
    "hisparse swap-in": "known-answer LRU trace (test_hisparse.py:108-129); exactness invariant "
    "(:65-90); 200-step golden trace from the reference (tests/golden)",
}
