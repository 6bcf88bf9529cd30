"""Latest Exact Match Attention on AMD MI355X (gfx950): the hot path of
moritzbroe/latest_exact_match_attention as hand-written HIP kernels behind the reference's
Python API.

    pack_codes(z)                    code/lema/attention.py:82
    latest_prev_match(qc, kc)        code/lema/attention.py:100
    lema_hard(q, k, v, store=None)   code/lema/attention.py:135

Every op runs on the GPU through liblema_hip.so (C ABI: include/lema_hip.h); there is no CPU
fallback.
"""
from .attention import (code_dtype_for, gather_values, latest_prev_match, lema_from_codes,
                        lema_hard, pack_codes)

__all__ = ["pack_codes", "latest_prev_match", "lema_hard", "lema_from_codes", "gather_values",
           "code_dtype_for"]
