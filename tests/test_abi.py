"""The C ABI library without a GPU (CPU only): it loads, exports every entry point the header
declares, validates arguments on the host with the documented statuses, and the Python API
refuses CPU tensors instead of falling back to a CPU path."""
import re
from pathlib import Path

import pytest
import torch

from latest_exact_match_attention_amd import _lib, build

ROOT = Path(__file__).resolve().parents[1]


@pytest.fixture(scope="module")
def L():
    build.ensure_built()
    return _lib.lib()


def _declared():
    text = (ROOT / "include" / "lema_hip.h").read_text()
    return sorted(set(re.findall(r"\b(lema_[a-z_0-9]+)\s*\(", text)))


def test_header_and_binding_agree():
    assert _declared() == sorted(_lib.PROTOTYPES)


def test_library_exports_every_declared_symbol(L):
    for name in _declared():
        assert hasattr(L, name), name
    assert L.lema_abi_version() >= 1


def test_host_validation_statuses(L):
    assert L.lema_latest_prev_match(None, None, 3, 1, 1, None, 4, None) == _lib.BAD_ARG
    assert b"code_bytes" in L.lema_last_error()
    assert L.lema_pack_codes(None, 2, 1, 1, 1, 65, 0, 0, 0, None, 8, None) == _lib.BAD_ARG
    assert b"> 64" in L.lema_last_error()
    assert L.lema_pack_codes(None, 2, 1, 1, 1, 33, 0, 0, 0, None, 4, None) == _lib.BAD_ARG
    assert L.lema_pack_codes(None, 9, 1, 1, 1, 8, 0, 0, 0, None, 8, None) == _lib.BAD_ARG
    assert L.lema_hard(None, None, 8, None, 2, -1, 1, 1, 1, 0, 0, 0, None, 0, 0, 0, 0, None, 4,
                       None) == _lib.BAD_ARG
    assert L.lema_gather(None, 2, 1, 1, 1, 1, 0, 0, 0, None, 5, None, 0, 0, 0, 0,
                         None) == _lib.BAD_ARG
    # the MLP launch with its pre-norm: x, d, nw, eps, x_out, wg, wu, ldw, M, N, K, out, stream
    f = L.lema_skinny_norm_swiglu_bf16
    assert f(256, 512, 768, 1e-5, 1024, 1280, 1536, 64, 33, 64, 64, 1792, None) == _lib.BAD_ARG
    assert f(256, 512, 768, 1e-5, 256, 1280, 1536, 64, 4, 64, 64, 1792, None) == _lib.BAD_ARG
    assert b"neither input" in L.lema_last_error()
    assert f(256, 512, 768, 1e-5, 1024, 1280, 1536, 2080, 4, 64, 2080, 1792, None) == _lib.BAD_ARG
    assert b"at most 2048" in L.lema_last_error()
    assert f(256, 512, 768, 1e-5, 1024, 1280, 1536, 2048, 32, 64, 2048, 1792, None) == _lib.BAD_ARG
    assert b"LDS" in L.lema_last_error()
    # prefill q/k codes: x, ldx, wq, wk, ldw, M, N, K, d, T, qcodes, kcodes, code_bytes, stream
    # (null pointers: the shape is refused before any pointer is looked at);
    # M rows x N / d heads x 4 bytes = 2^31 bytes of codes per projection, one past the limit
    # (M is not a multiple of d here, so the size is M * (N / d), not M / d * N)
    q = L.lema_qk_pack_bf16
    assert q(None, 1536, None, None, 1536, 8388608, 1536, 1536, 24, 16384, None, None, 4,
             None) == _lib.BAD_ARG
    assert b"2 GiB" in L.lema_last_error()
    assert q(None, 1536, None, None, 1536, 8386560, 1536, 1536, 24, 16384, None, None, 4,
             None) == _lib.BAD_ARG
    assert b"whole streams" in L.lema_last_error()  # the size passes; T does not divide M
    assert L.lema_argmax_bf16(256, 2, 7, 8, 512, 1, None) == _lib.BAD_ARG
    assert L.lema_embedding_bf16(256, 10, 12, 512, 3, 768, None) == _lib.BAD_ARG
    # empty work is a no-op that touches no pointer
    assert L.lema_latest_prev_match(None, None, 8, 0, 5, None, 8, None) == _lib.OK
    assert L.lema_pack_codes(None, 2, 0, 4, 4, 8, 0, 0, 0, None, 8, None) == _lib.OK


@pytest.mark.parametrize("P,T,bulk", [
    (24, 1024, False), (24, 1025, True), (128, 2048, True), (129, 2048, False),
    (129, 2049, True), (4096, 2048, False), (4096, 2049, True), (4096, 16384, True),
    (1, 1, False)])
def test_store_workspace_only_where_bulk_is_faster(L, P, T, bulk):
    """A store workspace (the bulk path) is asked for exactly where the bulk path was the
    faster one in measurement: T > 1024 up to 128 partitions, T > 2048 beyond."""
    for cb in (4, 8):
        assert (L.lema_store_workspace_bytes(P * T, T, cb) > 0) == bulk, (P, T, cb)
    assert L.lema_store_workspace_bytes(P * T, T, 2) == 0


def test_status_mapping():
    with pytest.raises(RuntimeError, match="full"):
        _lib.check(_lib.TABLE_FULL)


def test_python_api_refuses_cpu_tensors():
    from latest_exact_match_attention_amd import latest_prev_match, lema_hard, pack_codes
    q = torch.randn(1, 2, 8, 4)
    with pytest.raises(TypeError, match="HIP"):
        pack_codes(q)
    with pytest.raises(TypeError, match="HIP"):
        latest_prev_match(torch.zeros(2, 8, dtype=torch.int64),
                          torch.zeros(2, 8, dtype=torch.int64))
    with pytest.raises(TypeError, match="HIP"):
        lema_hard(q, q, q)
    with pytest.raises(ValueError, match="> 64"):
        pack_codes(torch.randn(2, 65))


def test_widen_codes_zero_extends_int32():
    """Mixed-width calls widen int32 codes to the int64 code with the same 32-bit pattern,
    which is what the kernels read (an unsigned word), never the sign-extended value."""
    t = torch.tensor([-7, -1, 0, 5, -(1 << 31)], dtype=torch.int32)
    got = _lib.widen_codes(t).tolist()
    assert got == [(1 << 32) - 7, (1 << 32) - 1, 0, 5, 1 << 31]
    w = torch.tensor([-7, 1 << 40], dtype=torch.int64)
    assert _lib.widen_codes(w) is w


def test_noalloc_scratch_size_agrees_with_header():
    text = (ROOT / "include" / "lema_hip.h").read_text()
    m = re.search(r"#define LEMA_NOALLOC_SCRATCH_BYTES \((\d+)LL \* 1024 \* 1024\)", text)
    assert m and int(m.group(1)) * 1024 * 1024 == _lib.NOALLOC_SCRATCH_BYTES
