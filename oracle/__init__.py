"""CPU oracle for the LEMA hot path -- TEST INFRASTRUCTURE ONLY.

Only `tests/`, `__graft_entry__.smoke()` and the CPU-baseline leg of `bench.py` import this
package, and only as the oracle of the parity checks or as the timed CPU counterpart. The product
(`latest_exact_match_attention_amd`) never imports it and has no CPU fallback.

Contents:
  * `liblema_oracle.so` (built from `lema_oracle.c` by `oracle/Makefile`) through ctypes:
    pack_codes, latest_prev_match (dictionary rule), gather, store_exchange;
  * pure-Python restatements for small inputs: the dictionary rule of
    verification/lema.py:19-33, an O(T^2) brute force, and a per-partition dict store
    (code/tests/test_store.py:17-41);
  * `ref_store()`: the reference's own C++ store (code/lema/csrc/store.cpp) compiled into
    `oracle/_ref/` where the reference sources were available at build time.
"""
from .oracle import *  # noqa: F401,F403
