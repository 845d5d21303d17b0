"""The C-ABI library loads and exports exactly what include/cortex_hip.h declares (CPU only).

No kernel is launched: only symbol checks and argument-validation paths that
return before touching the HIP runtime.
"""

from __future__ import annotations

import ctypes
import re
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "cortex_hip.h"


def _declared() -> dict[str, int]:
    """name -> number of parameters, parsed from the header."""
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    out = {}
    for m in re.finditer(r"\b(?:int|int64_t|const char\*)\s+(cortex_\w+)\s*\(([^)]*)\)\s*;", text):
        params = [p for p in m.group(2).split(",") if p.strip() and p.strip() != "void"]
        out[m.group(1)] = len(params)
    return out


def test_header_declares_entry_points():
    names = _declared()
    for must in ("cortex_pack_plan", "cortex_tokenize", "cortex_quantize_int8", "cortex_norm_linear",
                 "cortex_attention", "cortex_row_stats", "cortex_layer_norm", "cortex_last_error"):
        assert must in names


def test_library_exports_every_declared_symbol():
    from cortex import _native as nat

    lib = nat.load()
    for name in _declared():
        assert hasattr(lib, name), name


def test_binding_signatures_match_header():
    from cortex import _native as nat

    decl = _declared()
    assert set(decl) == set(nat.EXPORTED)
    for name, (_, args) in nat._SIGNATURES.items():
        assert len(args) == decl[name], (name, len(args), decl[name])


def test_invalid_arguments_return_status_and_message():
    from cortex import _native as nat

    lib = nat.load()
    assert lib.cortex_version() == 1
    rc = lib.cortex_quantize_int8(None, -1, 4, 4, None, None, None, 4, None)
    assert rc == -1 and b"negative shape" in lib.cortex_last_error()
    # a K split that does not divide K (no pointer is dereferenced before the check)
    rc = lib.cortex_linear_residual_splitk(256, 512, 2048, 16, 2048, 16, 2048, None, None, 16, 512, 0, 16, 512, 3,
                                           16, 1 << 30, None)
    assert rc == -1 and b"multiple of 64 * splits" in lib.cortex_last_error()
    rc = lib.cortex_attention(1, 1, 1, 1, 1, 0, *([None, 0, 0, 0] * 3), None, None, None, 0, None, 0, 0, 0, 0, 0,
                              ctypes.c_float(1.0), None, 0, 0, 0, None)
    assert rc == -1 and b"head dim" in lib.cortex_last_error()
    rc = lib.cortex_norm_linear(4, 4, 4, 0, None, 4, 0, None, None, None, 0, 1, 3, 0, None, 4, None, 0, None, 0, 0,
                                None, 0, 0, 0, None, 4, None)
    assert rc == -1
    assert lib.cortex_pack_workspace_bytes(0, 4) == 0
    # five 1024-event chunks of 32 counts, then one status word per 256 events
    assert lib.cortex_pack_workspace_bytes(5000, 32) == (5 * 32 + 20) * 4
    rc = lib.cortex_pack_plan(None, 1, 10, 100000, None, None, None, None, None, 0, None, None, 0, None)
    assert rc == -1 and b"exceeds" in lib.cortex_last_error()
    # widening riders: at most 8 arrays, counts in multiples of 16, 16-byte aligned arrays
    src = (ctypes.c_void_p * 9)(*([16] * 9))
    cnt = (ctypes.c_int64 * 9)(*([16] * 9))
    rc = lib.cortex_widen_int8(9, src, src, cnt, None, None)
    assert rc == -1 and b"at most 8" in lib.cortex_last_error()
    cnt[0] = 24
    rc = lib.cortex_widen_int8(1, src, src, cnt, None, None)
    assert rc == -1 and b"multiple of 16" in lib.cortex_last_error()
    cnt[0], src[0] = 16, 8
    rc = lib.cortex_ln_rows_widen(0, 512, None, 512, None, None, 1e-5, None, None, 0.0, None, 512, None, 512, 1, src,
                                  src, cnt, None, None)
    assert rc == -1 and b"16-byte aligned" in lib.cortex_last_error()
    assert lib.cortex_widen_int8(0, None, None, None, None, None) == 0
    cnt[0], src[0] = 16 * 96, 16
    fk = (ctypes.c_int64 * 1)(96)  # a fragment-order K must be a power of two
    rc = lib.cortex_widen_int8(1, src, src, cnt, fk, None)
    assert rc == -1 and b"power of two" in lib.cortex_last_error()
    # the fragment-order weight: 16-row, 32-K blocks; the direct-weight kernel takes K 256 / 512
    rc = lib.cortex_frag_weight(24, 64, 16, 1, 64, 16, None)
    assert rc == -1 and b"multiple of 16" in lib.cortex_last_error()
    rc = lib.cortex_linear_residual_ln(64, 512, 128, 16, 128, 7, 16, 128, None, None, 16, 512, 0, 16, 512, 16, 16,
                                       ctypes.c_float(1e-5), 16, 512, None)
    assert rc == -1 and b"K = 256 or 512" in lib.cortex_last_error()


def test_missing_library_fails_loudly(monkeypatch, tmp_path):
    import importlib

    from cortex import _native as nat

    monkeypatch.setenv("CORTEX_HIP_LIB", str(tmp_path / "nope.so"))
    fresh = importlib.reload(nat)
    try:
        with pytest.raises(fresh.NativeLibraryError):
            fresh.load()
        assert not fresh.available()
    finally:
        monkeypatch.delenv("CORTEX_HIP_LIB")
        importlib.reload(nat)
