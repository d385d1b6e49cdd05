"""The C-ABI library loads (no GPU needed) and exports every entry point the
header declares; the Python binding declares exactly those symbols."""
import ctypes
import os
import re

import pytest

from nanovllm_amd import _native

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "nanovllm_amd.h")


def declared_symbols():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(nva_\w+)\s*\(", text)))


def test_header_declares_the_hot_path_entry_points():
    syms = declared_symbols()
    for name in ("nva_store_kvcache", "nva_store_kvcache_paged", "nva_rollback", "nva_aux_gather", "nva_argmax_accept",
                 "nva_argmax_rows", "nva_paged_attention_varlen", "nva_paged_attention_decode"):
        assert name in syms


def test_library_exports_every_declared_symbol():
    if not os.path.exists(_native.LIB_PATH):
        pytest.fail(f"{_native.LIB_PATH} missing: run __graft_entry__.build()")
    lib = ctypes.CDLL(_native.LIB_PATH)
    missing = [s for s in declared_symbols() if not hasattr(lib, s)]
    assert not missing, missing


def test_binding_covers_the_header():
    assert sorted(_native.SIGNATURES) == declared_symbols()


_C_TYPES = {"int32_t": ctypes.c_int32, "int64_t": ctypes.c_int64, "int": ctypes.c_int,
            "float": ctypes.c_float, "size_t": ctypes.c_size_t}


def header_signatures():
    """(restype, argtypes) of every declaration in the header, from its C
    parameter types: pointers are c_void_p (c_char_p for a returned string)."""
    text = re.sub(r"/\*.*?\*/", "", open(HEADER).read(), flags=re.S)
    sigs = {}
    for ret, name, params in re.findall(r"([\w ]+?\s*\*?)\s*\b(nva_\w+)\s*\(([^)]*)\)\s*;", text):
        ret = ret.strip()
        restype = ctypes.c_char_p if "char" in ret and "*" in ret else _C_TYPES[ret.split()[-1]]
        args = []
        for prm in params.split(","):
            prm = prm.strip()
            if prm in ("", "void"):
                continue
            args.append(ctypes.c_void_p if "*" in prm else _C_TYPES[prm.split()[-2]])
        sigs[name] = (restype, args)
    return sigs


def test_binding_matches_the_header_types():
    sigs = header_signatures()
    assert sorted(sigs) == declared_symbols()
    for name, (restype, argtypes) in _native.SIGNATURES.items():
        assert sigs[name] == (restype, argtypes), name


def test_integration_doc_argtypes_match_the_header():
    """Every `_lib.nva_*.argtypes = [...]` line of the integration guide's
    ctypes snippets declares the header's parameter types."""
    doc = open(os.path.join(ROOT, "INTEGRATION.md")).read()
    names = {"P": ctypes.c_void_p, "I32": ctypes.c_int32, "I64": ctypes.c_int64,
             "INT": ctypes.c_int, "F32": ctypes.c_float, "SZ": ctypes.c_size_t}
    found = re.findall(r"_lib\.(nva_\w+)\.argtypes\s*=\s*(\[[^\]]*\](?:\s*\*\s*\d+)?)", doc)
    assert len(found) >= 10
    for name, expr in found:
        argtypes = eval(expr, {"__builtins__": {}}, names)
        assert argtypes == _native.SIGNATURES[name][1], name


def test_host_side_argument_errors_without_gpu():
    lib = _native.load()
    assert lib.nva_version().startswith(b"nanovllm_amd")
    # bad arguments are rejected on the host before any launch
    assert lib.nva_store_kvcache(None, 0, None, 0, None, None, 7, None, 4, 1, 128, 10,
                                 None, None, None) == _native.NVA_ERR_ARG
    assert lib.nva_store_kvcache_paged(None, 0, None, 0, None, None, 0, 0, 0, 0, 1, 0, None, 4,
                                       1, 128, None, None, None) == _native.NVA_ERR_ARG
    assert lib.nva_aux_gather(None, None, 9, 0, 0, 0, None, 1, None, 0, None) == _native.NVA_ERR_ARG
    assert lib.nva_paged_attention_decode(None, 0, 0, None, None, 0, 0, 0, 0, 1, 256, None, None,
                                          0, 1, 1, 16, 8, 8, 64, 1.0, None, None, None, 0, 0,
                                          None, 0, None) == _native.NVA_ERR_UNSUPPORTED
    assert lib.nva_argmax_accept(None, 10, 5, None, 1, 1, None, None, None, None, None, 0,
                                 None) == _native.NVA_ERR_ARG
    # the allocation-free argmax refuses more chunk keys than its static
    # array holds on the host (the pointers are never touched): 6554 rows of
    # ten 16384-element chunks need 65540 keys; 6553 rows would fit
    fake = 4096
    assert _native.ARGMAX_STATIC_KEYS == 65536
    assert lib.nva_argmax_accept_static(fake, 151936, 151936, fake, 1, 6554, fake, fake, fake,
                                        fake, None) == _native.NVA_ERR_CAPACITY
    assert lib.nva_argmax_accept_static(None, 10, 5, None, 1, 1, None, None, None, None,
                                        None) == _native.NVA_ERR_ARG
    with pytest.raises(ValueError, match="static scratch capacity"):
        _native.check(_native.NVA_ERR_CAPACITY, "probe")
    # commit metadata: a zero verify stride, a missing accept buffer and more
    # sequences than the one-workgroup scan holds are refused on the host
    assert lib.nva_commit_metadata(fake, fake, 2, 0, fake, 12, fake, 4, 4, 256, 0, fake, fake,
                                   fake, fake, fake, fake, fake, 12, None) == _native.NVA_ERR_ARG
    assert lib.nva_commit_metadata(fake, None, 2, 6, fake, 12, fake, 4, 4, 256, 0, fake, fake,
                                   fake, fake, fake, fake, fake, 12, None) == _native.NVA_ERR_ARG
    assert lib.nva_commit_metadata(fake, fake, 2049, 6, fake, 12, fake, 4, 4, 256, 0, fake, fake,
                                   fake, fake, fake, fake, fake, 12,
                                   None) == _native.NVA_ERR_UNSUPPORTED
    # the draft slot convention is 0 (slot p) or 1 (the reference's slot
    # p + 1); any other offset is refused by both draft-side entries
    for off in (-1, 2):
        assert lib.nva_commit_metadata(fake, fake, 2, 6, fake, 12, fake, 4, 4, 256, off, fake,
                                       fake, fake, fake, fake, fake, fake, 12,
                                       None) == _native.NVA_ERR_ARG
        assert lib.nva_draft_metadata(fake, fake, fake, 2, 4, 3, fake, 4, 4, 256, off, fake,
                                      fake, fake, None) == _native.NVA_ERR_ARG
    # zero-size work is a no-op
    assert lib.nva_argmax_rows(None, 8, 8, 0, None, None, None, 0, None) == _native.NVA_OK
    assert lib.nva_argmax_workspace_size(384, 64, 151936) > 0
    assert lib.nva_paged_attention_workspace_size(64, 384, 32, 8, 128, 6, 2304) > 0
    with pytest.raises(ValueError):
        _native.check(_native.NVA_ERR_ARG, "probe")
    with pytest.raises(_native.KernelError):
        _native.check(_native.NVA_ERR_LAUNCH, "probe")


def test_attention_workspace_covers_every_layout():
    """The workspace size query names no KV dtype, so it must cover the
    largest layout either dtype can pick: for single-tile batches of 17-32
    rows that is the FP8 stream decomposition (split count bound: one per 4
    chunks of 32 keys, plus one), even when bf16 would run unsplit."""
    lib = _native.load()
    seqs, tokens, hq, hkv, max_q, max_k = 16, 96, 32, 8, 6, 2310
    got = lib.nva_paged_attention_workspace_size(seqs, tokens, hq, hkv, 128, max_q, max_k)
    chunks = -(-max_k // 32)
    splits = (chunks + 3) // 4 + 1
    slots = tokens * hq * splits
    need = slots * 128 * 4 + slots * 4 + tokens * 4
    assert got >= need, (got, need)
    # a bf16-only shape: no split at all needs no workspace beyond zero
    assert lib.nva_paged_attention_workspace_size(64, 384, 32, 8, 128, 6, 1024) >= 0
