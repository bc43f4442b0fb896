"""The C ABI library without a GPU: it loads, exports every function include/llmserve_hip.h
declares, and its argument checks (the reference's TORCH_CHECKs) reject bad calls before
anything is launched."""

from __future__ import annotations

import re

import pytest

from conftest import REPO

HEADER = REPO / "include" / "llmserve_hip.h"


def declared_functions() -> list[str]:
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    return re.findall(r"\b(llmserve_\w+)\s*\(", text)


@pytest.fixture(scope="module")
def lib():
    from llmserve._native import capi

    return capi()


def test_every_declared_symbol_is_exported_and_typed(lib):
    from llmserve._native import C_SIGNATURES

    names = declared_functions()
    assert len(names) >= 9
    for n in names:
        assert hasattr(lib, n), n
        assert n in C_SIGNATURES, f"{n} has no ctypes signature"
    assert set(C_SIGNATURES) == set(names)
    assert lib.llmserve_abi_version() == 1


def _err(lib) -> str:
    return lib.llmserve_last_error().decode()


def test_gemv_argument_checks(lib):
    assert lib.llmserve_int8_linear(None, None, None, None, 65, 8, 16, None) == 1
    assert "M <= 64" in _err(lib)
    assert lib.llmserve_int8_linear(None, None, None, None, 0, 8, 16, None) == 0  # empty: no launch
    assert lib.llmserve_int8_linear(None, None, None, None, 2, 8, 16, None) == 1
    assert "null pointer" in _err(lib)
    assert lib.llmserve_int4_linear(None, None, None, None, None, None, 1, 8, 100, 64, None) == 1
    assert "int4: shapes" in _err(lib)
    assert lib.llmserve_int4_linear(None, None, None, None, None, None, 1, 8, 96, 3, None) == 1


def test_quantizer_argument_checks(lib):
    assert lib.llmserve_int4_quantize(None, None, None, None, None, None, 4, 100, 64, None) == 1
    assert "not divisible by group" in _err(lib)
    assert lib.llmserve_int4_quantize(None, None, None, None, None, None, 4, 99, 33, None) == 1
    assert lib.llmserve_int8_quantize(None, None, None, 0, 16, None) == 0
    assert lib.llmserve_kv_quantize_write(None, None, None, None, None, 0, 2, 32, 64, None) == 0


def test_paged_attention_argument_checks(lib):
    f = lib.llmserve_paged_attention_decode_int8
    args = [None] * 8
    assert f(*args, 2, 6, 4, 32, 64, 4, 4, 0.1, 0, None, None, 0, None) == 1
    assert "multiple of Hk" in _err(lib)
    assert f(*args, 0, 8, 4, 32, 64, 4, 4, 0.1, 0, None, None, 0, None) == 0  # B == 0
    assert f(*args, 2, 8, 4, 48, 64, 4, 4, 0.1, 0, None, None, 0, None) == 1
    assert "head_dim" in _err(lib)
    assert f(*args, 2, 72, 4, 32, 64, 4, 4, 0.1, 0, None, None, 0, None) == 1
    assert "at most 8" in _err(lib)


def test_paged_attention_workspace_size(lib):
    ws = lib.llmserve_paged_attention_workspace_bytes

    def expect(B, Hq, Hk, D, max_blocks, bs, P, HB):
        # ranges * HB partial slots of G (m, l, acc[D]) rows; with a fixed range size every
        # (b, head group) unit has at most ceil(max_blocks * bs / P) ranges (ranges never
        # straddle two units)
        nhg, G = Hk // HB, Hq // Hk
        ranges = B * nhg * -(-max_blocks * bs // P)
        return ranges * HB * G * (D + 2) * 4 + B * nhg * 4  # + each unit's range count

    # 8 kv heads share a workgroup; one range covers a whole unit
    assert ws(4, 16, 8, 128, 4, 16, 10_000) == expect(4, 16, 8, 128, 4, 16, 10_000, 8)
    # 32-token ranges over 256-token units: 8 per unit, 16 ranges
    assert ws(2, 16, 8, 128, 16, 16, 32) == expect(2, 16, 8, 128, 16, 16, 32, 8)
    # 6 kv heads: groups of 6
    assert ws(1, 12, 6, 64, 2, 16, 16) == expect(1, 12, 6, 64, 2, 16, 16, 6)
    # 16 kv heads: two groups of 8
    assert ws(3, 32, 16, 64, 5, 16, 40) == expect(3, 32, 16, 64, 5, 16, 40, 8)
    assert ws(0, 16, 8, 128, 16, 16, 32) == 0
    # the balanced plan (P = 0) bounds each unit's slots by a multiple of its share of the
    # grid, so a large batch's workspace does not grow with the context bound, and stays
    # within the fixed 64-token split's
    assert ws(256, 32, 8, 128, 2048, 16, 0) == ws(256, 32, 8, 128, 4096, 16, 0)
    assert ws(256, 32, 8, 128, 2048, 16, 0) < ws(256, 32, 8, 128, 2048, 16, 64)
    assert ws(1, 32, 8, 128, 64, 16, 0) <= ws(1, 32, 8, 128, 64, 16, 64)


def test_single_hip_runtime_with_torch():
    """The library binds to the HIP runtime torch loaded (both are libamdhip64.so.7)."""
    import torch  # noqa: F401

    from llmserve._native import capi, ops

    ops()
    capi()
    maps = {line.split()[-1] for line in open("/proc/self/maps") if "libamdhip64" in line}
    assert len(maps) == 1, maps
