"""MI355X (gfx950) beam-aware KV-cache path: BeamAttention decode, beam KV
fork/append and fused beam pruning behind vLLM-GR's attention-backend and
beam-search plugin interfaces.

The compute lives in ``_lib/libgr_beam.so`` (hand-written HIP, C ABI in
``include/gr_beam.h``); ``ops`` wraps it for torch tensors.
"""

__version__ = "0.1.0"
