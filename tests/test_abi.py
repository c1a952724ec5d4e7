"""C ABI: libsrswa.so loads, exports every function include/srswa.h declares,
and the ctypes argument structs match the header field for field.  No kernel
is launched (CPU-only)."""

import ctypes
import os
import re

import srswa
from srswa import _lib

HEADER = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))),
                      "include", "srswa.h")


def _header_text():
    src = open(HEADER).read()
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    return re.sub(r"//[^\n]*", "", src)


def _declared_functions():
    return set(re.findall(r"^\s*(?:const\s+)?[\w\s\*]*?\b(srswa_\w+)\s*\(", _header_text(), flags=re.M))


_CTYPES = {"int64_t": ctypes.c_int64, "int32_t": ctypes.c_int32, "float": ctypes.c_float,
           "double": ctypes.c_double}


def _declared_structs():
    """{struct name: [(field, ctypes type), ...]} from the header (pointers -> c_void_p)."""
    out = {}
    for body, name in re.findall(r"typedef\s+struct\s*\{(.*?)\}\s*(\w+)\s*;", _header_text(), flags=re.S):
        fields = []
        for decl in body.split(";"):
            decl = decl.strip()
            if not decl:
                continue
            m = re.match(r"(const\s+)?([\w]+)\s*(.*)", decl)
            base = m.group(2)
            for n in m.group(3).split(","):
                n = n.strip()
                ty = ctypes.c_void_p if n.startswith("*") else _CTYPES[base]
                fields.append((n.lstrip("*").strip(), ty))
        out[name] = fields
    return out


def test_library_loads_and_exports_every_declared_symbol():
    lib = _lib.lib()
    declared = _declared_functions()
    assert declared, "no functions parsed from the header"
    for name in declared:
        assert hasattr(lib, name), f"{name} declared in srswa.h but not exported"
    assert set(_lib.SIGNATURES) == declared, set(_lib.SIGNATURES) ^ declared
    assert lib.srswa_version() >= 100


def test_ctypes_structs_match_header():
    structs = _declared_structs()
    assert set(structs) == set(_lib.STRUCTS), set(structs) ^ set(_lib.STRUCTS)
    for cname, fields in structs.items():
        py = [(f[0], f[1]) for f in _lib.STRUCTS[cname]._fields_]
        assert py == fields, (cname, py, fields)


def test_workspace_query_needs_no_gpu():
    a = _lib.DecodeArgs()
    a.B, a.Lq, a.HQ, a.HKV, a.HI, a.D, a.S, a.L = 64, 1, 10, 10, 10, 128, 8, 131072
    a.block_size, a.local_window, a.in_dtype, a.out_dtype = 64, 512, _lib.SRSWA_BF16, _lib.SRSWA_BF16
    scr = _lib.lib().srswa_gather_decode_workspace(ctypes.byref(a))
    # 640 (row, head) pairs x 4 workgroups x 160-float records
    assert scr == 640 * 4 * 160 * 4
    assert srswa.__version__


def _hc_args(cls, **over):
    """head_cls scorer arguments with dummy 16-byte-aligned device addresses
    (never dereferenced: every case below is refused before any launch)."""
    a = cls()
    B, S, D, nblk = 2, 1024, 128, 16
    for i, name in enumerate(n for n, _ in cls._fields_ if n in ("q", "k", "head_cls", "pos", "kbar", "z", "gz",
                                                                     "dq", "dk", "dhc")):
        setattr(a, name, 0x100000 * (i + 1))
    a.B, a.S, a.D, a.nblk, a.block_size, a.local_blocks = B, S, D, nblk, 64, 8
    a.q_sb, a.q_st, a.k_sb, a.k_st = S * D, D, S * D, D
    a.pos_sb, a.pos_st, a.kb_sb, a.z_sb, a.z_st = S, 1, nblk * D, S * nblk, nblk
    if cls is _lib.HcScoreBwdArgs:
        a.gz_sb, a.gz_st, a.dq_sb, a.dq_st, a.dk_sb, a.dk_st = S * nblk, nblk, S * D, D, S * D, D
    for k, v in over.items():
        setattr(a, k, v)
    return a


def test_hc_scores_refuse_overlapping_or_huge_rows():
    """The head_cls scorers address z / gz / q tiles through buffer resources
    with 32-bit offsets: overlapping rows and strides of 2^23 or more are
    refused with SRSWA_UNSUPPORTED on the host (no GPU needed), and so are
    q / k / dq / dk rows that are not 16-byte aligned (read and written as
    float4)."""
    lib = _lib.lib()
    assert lib.srswa_hc_score_fwd(ctypes.byref(_hc_args(_lib.HcScoreArgs, z_st=8)), None) == _lib.SRSWA_UNSUPPORTED
    assert lib.srswa_hc_score_fwd(ctypes.byref(_hc_args(_lib.HcScoreArgs, z_st=1 << 23, z_sb=1 << 34)),
                                  None) == _lib.SRSWA_UNSUPPORTED
    for over in (dict(z_st=8), dict(gz_st=8), dict(q_st=64, k_st=128), dict(gz_st=1 << 23, gz_sb=1 << 34),
                 dict(dk=0x100004), dict(dk_st=130), dict(dk_sb=1024 * 128 + 2), dict(k_st=129)):
        a = _hc_args(_lib.HcScoreBwdArgs, **over)
        need = ctypes.c_size_t()
        assert lib.srswa_hc_score_bwd_workspace(ctypes.byref(a), ctypes.byref(need)) == _lib.SRSWA_OK
        rc = lib.srswa_hc_score_bwd(ctypes.byref(a), ctypes.c_void_p(0x4000000), need.value, None)
        assert rc == _lib.SRSWA_UNSUPPORTED, over
