"""The C-ABI library loads and exports every entry point include/nq_abi.h declares (no GPU needed)."""

from __future__ import annotations

import ctypes
import re
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "nq_abi.h"


def _declared() -> set[str]:
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return set(re.findall(r"\b(nq_[a-z0-9_]+)\s*\(", text))


def test_header_and_binding_agree(nq):
    from nari_qwen3_tts_amd import _lib

    assert _declared() == set(_lib.EXPORTED)


def _declared_parameters() -> dict[str, list[str]]:
    """name -> the C types of its parameters, as include/nq_abi.h declares them."""

    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    text = re.sub(r"//[^\n]*", "", text)
    out = {}
    for m in re.finditer(r"\b(nq_[a-z0-9_]+)\s*\(([^)]*)\)\s*;", text):
        params = [q.strip() for q in m.group(2).replace("\n", " ").split(",") if q.strip()]
        if params == ["void"]:
            params = []
        # drop the parameter name: the type is everything before it
        out[m.group(1)] = [re.sub(r"\s*\b[a-zA-Z_][a-zA-Z0-9_]*$", "", q) if not q.endswith("*") else q
                           for q in params]
    return out


def _ctype_of(c_type: str):
    c_type = c_type.replace("const ", "").strip()
    if "*" in c_type:
        return ctypes.c_void_p
    return {"int": ctypes.c_int, "int64_t": ctypes.c_int64, "float": ctypes.c_float}[c_type]


def test_binding_argument_types_match_the_header(nq):
    """Every ctypes signature has the header's arity and argument kinds (pointer / int / int64 /
    float), so a parameter added to one side but not the other fails here, on the CPU, instead of
    passing a shifted argument list to the library."""
    from nari_qwen3_tts_amd import _lib

    declared = _declared_parameters()
    assert set(declared) == set(_lib.EXPORTED)
    for name, params in declared.items():
        want = [_ctype_of(t) for t in params]
        got = _lib._SIGNATURES[name]
        assert len(got) == len(want), (name, len(got), len(want))
        assert got == want, (name, [t.__name__ for t in got], [t.__name__ for t in want])


def test_library_exports_every_declared_symbol(nq):
    from nari_qwen3_tts_amd import _lib

    if not _lib.LIBRARY_PATH.exists():
        pytest.fail("libnq_hip.so is not built; run __graft_entry__.build()")
    lib = ctypes.CDLL(str(_lib.LIBRARY_PATH))
    for name in _declared():
        assert hasattr(lib, name), name


def test_host_side_metadata_queries_need_no_gpu(nq):
    from nari_qwen3_tts_amd import _lib

    lib = _lib.load()
    assert lib.nq_abi_version() == 1
    assert _lib.status_string(-4) == "not enough free KV pages"
    assert lib.nq_attention_workspace_bytes(64, 32832, 16, 16, 8, 128) > 0
    assert lib.nq_attention_workspace_bytes(0, 1, 16, 16, 8, 128) == -1


def test_argument_errors_are_caught_on_the_host(nq):
    """Invalid shapes return NQ_ERR_* before anything is launched."""

    from nari_qwen3_tts_amd import _lib

    lib = _lib.load()
    # capture rows above the single-workgroup limit
    assert lib.nq_plan_ragged(*([None] * 5), 1, 2048, 1, 16, 0, None, 1, None, 0, None, None, 2048, None, None, None,
                              0, None, None, None, None, None, 0, None) == -2
    # vocabulary above the sampler's LDS budget
    assert lib.nq_sample(1, 0, 8192, 1, 8192, 1, 1, 1, None, None, 0, 1, 8192, -1, None, 0, 1, None) == -2
    with pytest.raises(TypeError):
        _lib.check(-2, "x")
    with pytest.raises(ValueError):
        _lib.check(-1, "x")
    from nari_qwen3_tts_amd.errors import KVAllocationError

    with pytest.raises(KVAllocationError):
        _lib.check(-4, "x")


def test_attention_parts_flags(nq):
    """The attention part flags agree with the header, and flag sets without a part to run, with an
    unknown bit, or with the beside-prefill bit but no decode part are refused on the host."""

    from nari_qwen3_tts_amd import _lib

    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    body = re.search(r"enum nq_attention_parts \{([^}]*)\}", text).group(1)
    declared = {k.strip(): int(v) for k, v in (e.split("=") for e in body.split(",") if e.strip())}
    assert declared == {"NQ_ATTN_DECODE": _lib.NQ_ATTN_DECODE, "NQ_ATTN_PREFILL": _lib.NQ_ATTN_PREFILL,
                        "NQ_ATTN_BESIDE_PREFILL": _lib.NQ_ATTN_BESIDE_PREFILL}
    lib = _lib.load()

    def call(parts):
        # placeholder pointers: the argument checks run before any device access
        return lib.nq_paged_attention(1, 2048, 128, 1, 65536, 32768, 2048, 128, 64, 1, 16, 16, 8, 128, 0.088, 1,
                                      2048, 128, 64, 1024, parts, 1, 1 << 40, None, None)

    for parts in (0, _lib.NQ_ATTN_BESIDE_PREFILL, _lib.NQ_ATTN_PREFILL | _lib.NQ_ATTN_BESIDE_PREFILL, 8):
        assert call(parts) == -1, parts
    # accepted flag sets pass on to the next check, which refuses the misaligned placeholder pointers
    for parts in (_lib.NQ_ATTN_DECODE, _lib.NQ_ATTN_DECODE | _lib.NQ_ATTN_BESIDE_PREFILL,
                  _lib.NQ_ATTN_DECODE | _lib.NQ_ATTN_PREFILL):
        assert call(parts) == -2, parts
