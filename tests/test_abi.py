"""The C ABI: the library loads on a host without a GPU and exports every symbol its header
declares (no compute calls here)."""

from __future__ import annotations

import ctypes
import os
import re

import pytest

from conftest import ROOT

HEADER = os.path.join(ROOT, "include", "mote_relation.h")


def _declared():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"^\s*(?:const\s+)?(?:int|size_t|char\s*\*|const char\s*\*)\s*\*?\s*(mote_\w+)\s*\(", text, re.M)))


def _header_structs():
    """{struct: [field, ...]} in declaration order, read from the header text."""
    text = re.sub(r"/\*.*?\*/", "", open(HEADER).read(), flags=re.S)
    out = {}
    for m in re.finditer(r"typedef struct (\w+) \{(.*?)\} \1;", text, re.S):
        fields = []
        for decl in filter(None, (d.strip() for d in m.group(2).split(";"))):
            first, *rest = decl.split(",")
            fields += [first.split()[-1].lstrip("*")] + [r.strip().lstrip("*") for r in rest]
        out[m.group(1)] = fields
    return out


def test_header_declares_the_entry_points():
    names = _declared()
    for n in ["mote_relation_fwd", "mote_relation_bwd", "mote_relation_bwd_workspace", "mote_relation_decode",
              "mote_relation_decode_workspace", "mote_rope_givens_fwd", "mote_rope_givens_bwd",
              "mote_rope_givens_bwd_workspace", "mote_last_error", "mote_version"]:
        assert n in names, n


def test_library_exports_every_declared_symbol():
    from mote_amd import _lib

    if not _lib.available():
        pytest.skip("libmote_relation.so not built")
    lib = ctypes.CDLL(_lib.LIB_PATH)
    missing = [n for n in _declared() if not hasattr(lib, n)]
    assert not missing, missing
    assert set(_lib.EXPORTS) == set(_declared())
    assert b"gfx950" in _lib.lib().mote_version()


def test_argument_errors_are_reported_without_a_gpu():
    """Validation happens before any launch: a bad dtype comes back as a status and a message."""
    from mote_amd import _lib

    if not _lib.available():
        pytest.skip("libmote_relation.so not built")
    a = _lib.FwdArgs()
    a.dtype = 7
    rc = _lib.lib().mote_relation_fwd(a, None)
    assert rc == 1
    assert b"dtype" in _lib.lib().mote_last_error()
    a.dtype = _lib.MOTE_BF16
    a.p1.data = a.p2.data = a.info.data = a.y.data = 16
    a.ibar = a.lse = a.g = a.lam = 16
    a.B, a.H, a.TQ, a.TK, a.D = 1, 1, 4, 4, 100
    assert _lib.lib().mote_relation_fwd(a, None) == 2
    assert b"head dim" in _lib.lib().mote_last_error()


def test_skinny_gemm_rejects_unsupported_shapes_without_a_gpu():
    """mote_skinny_gemm checks dtype, row count and the N / K granularity before any launch."""
    from mote_amd import _lib

    if not _lib.available():
        pytest.skip("libmote_relation.so not built")
    a = _lib.SkinnyGemmArgs()
    a.dtype, a.B, a.N, a.K = _lib.MOTE_F32, 1, 16, 128
    a.x = a.w = a.y = 16
    a.x_sr = a.w_sr = a.y_sr = 128
    assert _lib.lib().mote_skinny_gemm(a, None) == 1
    assert b"bf16" in _lib.lib().mote_last_error()
    a.dtype = _lib.MOTE_BF16
    for B, N, K in ((17, 16, 128), (1, 24, 128), (1, 16, 100), (1, 16, 2048)):
        a.B, a.N, a.K = B, N, K
        assert _lib.lib().mote_skinny_gemm(a, None) == 2, (B, N, K)
    a.B, a.N, a.K = 0, 16, 128
    assert _lib.lib().mote_skinny_gemm(a, None) == 0  # nothing to do, nothing launched


def test_wgrad_rejects_unsupported_arguments_without_a_gpu():
    """mote_wgrad checks dtype, the 128-granular widths, strides, alignment and the workspace
    before any launch; its workspace query sizes the fp32 split partials (none for one split)."""
    from mote_amd import _lib

    if not _lib.available():
        pytest.skip("libmote_relation.so not built")
    a = _lib.WgradArgs()
    a.dtype, a.M, a.N, a.K = _lib.MOTE_F32, 64, 128, 128
    a.a = a.x = a.dw = 16
    a.a_sr = a.x_sr = a.dw_sr = 128
    assert _lib.lib().mote_wgrad(a, None) == 1
    assert b"bf16" in _lib.lib().mote_last_error()
    a.dtype = _lib.MOTE_BF16
    for M, N, K in ((-1, 128, 128), (64, 100, 128), (64, 128, 96), (64, 0, 128)):
        a.M, a.N, a.K = M, N, K
        assert _lib.lib().mote_wgrad(a, None) == 2, (M, N, K)
    a.M, a.N, a.K, a.a_sr = 64, 256, 128, 128  # a row stride below N
    assert _lib.lib().mote_wgrad(a, None) == 1
    a.a_sr, a.a = 256, 24  # a misaligned row start
    assert _lib.lib().mote_wgrad(a, None) == 1
    assert b"16-byte" in _lib.lib().mote_last_error()
    a.a = 16
    # a long reduction over few tiles splits M; every split holds an N x K fp32 partial
    a.M, a.N, a.K, a.a_sr, a.x_sr, a.dw_sr = 4964, 2304, 768, 2304, 768, 768
    ws = int(_lib.lib().mote_wgrad_workspace(a))
    assert ws > 0 and ws % (2304 * 768 * 4) == 0
    a.workspace, a.workspace_bytes = 16, ws - 16
    assert _lib.lib().mote_wgrad(a, None) == 3
    a.M = 200  # fewer than four stages per split: one split, no workspace
    assert int(_lib.lib().mote_wgrad_workspace(a)) == 0


def test_static_decode_refuses_shapes_beyond_its_array_without_a_gpu():
    """mote_relation_decode_static checks its arguments and the limits of its fixed scratch array
    (256 sequences, 1024 sequence-heads) before it touches a device: a larger call is refused with
    MOTE_ERR_WORKSPACE and a message naming the limits."""
    from mote_amd import _lib

    if not _lib.available():
        pytest.skip("libmote_relation.so not built")
    a = _lib.DecodeArgs()
    a.dtype = _lib.MOTE_BF16
    a.lam = a.S = a.p1 = a.p2 = a.info = a.y = a.g = 16
    a.cache_p2.data = a.cache_info.data = 16
    for B, H in ((257, 2), (130, 8), (64, 18)):  # too many sequences, sequence-heads
        a.B, a.H, a.D, a.capacity = B, H, 128, 4096
        assert _lib.lib().mote_relation_decode_static(a, None) == 3, (B, H)
        msg = _lib.lib().mote_last_error()
        assert f"B = {B} sequences x H = {H} heads".encode() in msg
        assert str(_lib.MOTE_DECODE_STATIC_BYTES).encode() in msg
    a.B, a.H = 128, 8
    a.D = 100
    assert _lib.lib().mote_relation_decode_static(a, None) == 2  # the shape checks come first
    a.D, a.g = 128, None
    assert _lib.lib().mote_relation_decode_static(a, None) == 1
    a.g = 16
    for slot in (-1, _lib.MOTE_DECODE_STATIC_SLOTS):  # a slot outside the array
        a.static_slot = slot
        assert _lib.lib().mote_relation_decode_static(a, None) == 1, slot
        assert f"static_slot = {slot}".encode() in _lib.lib().mote_last_error()


def test_ctypes_mirrors_match_the_compiled_struct_layout():
    """Every struct of the header: the library's table names the header's fields in order, and the
    ctypes mirror in mote_amd/_lib.py has the same size and the same offset and size per field."""
    from mote_amd import _lib

    if not _lib.available():
        pytest.skip("libmote_relation.so not built")
    layout = _lib.abi_layout()
    header = _header_structs()
    assert set(layout) == set(header) == set(_lib.STRUCTS)
    for name, fields in header.items():
        size, table = layout[name]
        assert list(table) == fields, name
        cls = _lib.STRUCTS[name]
        assert ctypes.sizeof(cls) == size, (name, ctypes.sizeof(cls), size)
        assert [f[0] for f in cls._fields_] == fields, name
        for f, (off, fsize) in table.items():
            desc = getattr(cls, f)
            assert (desc.offset, desc.size) == (off, fsize), (name, f, desc.offset, desc.size, off, fsize)
