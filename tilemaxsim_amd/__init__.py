"""tilemaxsim_amd -- fused MaxSim / PQ-ADC scoring on MI355X (gfx950 HIP kernels).

Drop-in host entry points for the reference modules ``src/flash_maxsim_v2.py``,
``src/flash_maxsim_kernel.py`` and ``src/flash_pqsim_kernel.py`` (plus the PLAID
drop-in of ``src/plaid_integration_benchmark.py``, the residual-compressed ColBERTv2
documents it scores, and the top-k its callers take); every
call runs hand-written HIP kernels from ``libtilemaxsim.so`` through its C ABI
(``include/tilemaxsim.h``). There is no CPU or PyTorch fallback.
"""
from .flash_maxsim_kernel import (flash_maxsim_batch, flash_maxsim_multi_doc, flash_maxsim_multi_doc_batched,
                                  flash_maxsim_single, maxsim_score)
from .flash_maxsim_v2 import flash_maxsim_batched_queries, flash_maxsim_v2, flash_maxsim_v2_multiquery
from .flash_pqsim_kernel import TileMaxSimPQ
from .plaid import flashmaxsim_score_packed, flashmaxsim_score_packed_batched
from .residual import decompress_residual, flashmaxsim_score_residual, flashmaxsim_score_residual_batched
from .topk import maxsim_topk, topk

__all__ = [
    "flash_maxsim_v2_multiquery", "flash_maxsim_v2", "flash_maxsim_batched_queries",
    "flash_maxsim_single", "flash_maxsim_batch", "flash_maxsim_multi_doc", "flash_maxsim_multi_doc_batched",
    "maxsim_score", "TileMaxSimPQ", "flashmaxsim_score_packed", "flashmaxsim_score_packed_batched", "topk",
    "maxsim_topk",
    "decompress_residual", "flashmaxsim_score_residual", "flashmaxsim_score_residual_batched",
]
