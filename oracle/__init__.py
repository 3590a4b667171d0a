"""CPU oracle for the beam-aware KV-cache path.  TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import anything from this package, and only as the checker
(or, for ``cpu_baseline``, as the timed CPU restatement of the reference).
The product path (``vllm_gr_amd``) never imports it and raises when its HIP
library is missing.

Modules (each function cites the reference file:line it restates):

* ``attention`` -- BeamAttention decode in float64 numpy over the build's
  resident-suffix layout: the dense per-beam form
  (``tests/kernels/attention/test_cascade_beam_flash_attn.py:191-319``) and
  the cascade form (prefix pass + suffix pass + LSE merge,
  ``vllm_gr/v1/attention/backends/beam_attn.py:629-701``).
* ``fork`` -- beam KV fork (copy-on-write block re-assignment by parent) and
  append; the child-suffix rule follows ``vllm_gr/v1/engine/core.py:108-112``
  and ``vllm_gr/entrypoints/openai/serving_engine.py:113-120``.
* ``prune`` -- fused log-softmax + cumulative logprob + top-k over
  beams x vocab (``serving_engine.py:457-592``, ``entrypoints/llm.py:201-280``),
  with the bit-exact numerics defined in ``prune_ref.c``.
* ``metadata`` -- the reference's own mega-request layout: the metadata
  builder's routing lists (``beam_attn.py:255-413``), the cascade over them
  (``:629-701``), and the reference kernel test's inputs and position-based
  reference (``test_cascade_beam_flash_attn.py:92-319``).
* ``sid_beam`` -- the end-to-end semantic-ID beam search: a float64 decoder
  forward and the reference's offline beam-search loop
  (``vllm_gr/entrypoints/llm.py:118-292``).

Pinning status of every function is listed in each module docstring.
"""
