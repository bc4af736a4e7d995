"""The C-ABI library loads, exports every declared symbol, and rejects bad
arguments with the documented codes before launching anything (no GPU
needed: validation runs on the host)."""
import ctypes
import glob
import os
import re

import pytest

from gmdn_amd import _native

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADERS = sorted(glob.glob(os.path.join(ROOT, "include", "*.h")))


def declared_functions():
    names = set()
    for h in HEADERS:
        text = re.sub(r"/\*.*?\*/", "", open(h).read(), flags=re.S)
        names |= set(re.findall(r"\b(gmdn_[a-z0-9_]+)\s*\(", text))
    return sorted(names)


def test_header_declares_expected_entry_points():
    names = declared_functions()
    for n in ("gmdn_scan_fwd", "gmdn_scan_bwd", "gmdn_chunk_fwd", "gmdn_chunk_bwd", "gmdn_error_string",
              "gmdn_front_fwd", "gmdn_front_bwd"):
        assert n in names


def test_library_exports_every_declared_symbol():
    lib = _native.load()
    for name in declared_functions():
        assert hasattr(lib, name), f"{name} missing from libgmdn_scan.so"
        assert name in _native.SIGNATURES, f"{name} has no ctypes signature"


def test_error_strings():
    lib = _native.load()
    for code in range(5):
        assert lib.gmdn_error_string(code)
    assert b"unknown" in lib.gmdn_error_string(99)


def test_supported_head_dims():
    lib = _native.load()
    assert [d for d in (16, 32, 48, 64, 128, 256) if lib.gmdn_scan_supported(d)] == [32, 64, 128]


def _fwd(lib, rule=0, dh=64, ns=3, prec=0, BH=2, N=3, null=()):
    p = [None if i in null else 0x1000 for i in range(9)]
    return lib.gmdn_scan_fwd(*p, BH, N, dh, rule, ns, prec, None)


def test_scan_fwd_argument_validation():
    lib = _native.load()
    assert _fwd(lib, rule=3) == 1
    assert _fwd(lib, ns=-1) == 1
    assert _fwd(lib, ns=9) == 1
    assert _fwd(lib, prec=2) == 1
    assert _fwd(lib, dh=48) == 2
    assert _fwd(lib, null=(0,)) == 1            # U
    assert _fwd(lib, null=(6,)) == 1            # S_all
    assert _fwd(lib, rule=1, null=(3,)) == 1    # muon needs b
    assert _fwd(lib, rule=2, null=(5,)) == 1    # adam needs n
    assert _fwd(lib, BH=0) == 0                 # empty problem: nothing to launch
    assert _fwd(lib, N=0) == 0


def test_scan_bwd_workspace_contract():
    lib = _native.load()
    assert lib.gmdn_scan_bwd_workspace_bytes(4, 16, 64, 0, 3) == 0
    assert lib.gmdn_scan_bwd_workspace_bytes(4, 16, 64, 2, 3) == 4 * 16 * 4 * 4 * 4
    # muon: per chunk of a segment 3 ns + 2 d x d matrices and |M_i|, per
    # (b, h) two carried matrices (at least the 4 + ns matrices per (b, h) of
    # the fp32 kernel); small problems are one segment of N chunks
    BH, N, mat = 4, 16, 64 * 64
    for ns in (1, 3, 5):
        x3 = BH * N * ((3 * ns + 2) * mat + 1) + 2 * BH * mat
        assert lib.gmdn_scan_bwd_workspace_bytes(BH, N, 64, 1, ns) == 4 * max(x3, BH * (4 + ns) * mat)
    assert lib.gmdn_scan_bwd_workspace_bytes(1, 1, 64, 1, 0) == 4 * max(2 * mat + 1 + 2 * mat, 4 * mat)
    # large problems: two buffers of segments of as many chunks as fit in
    # 512 MiB each
    BH, N, dh, ns = 32, 128, 128, 5
    per = BH * ((3 * ns + 2) * dh * dh + 1)
    nseg = ((512 << 20) // 4 - 2 * BH * dh * dh) // per
    assert 1 <= nseg < N
    assert lib.gmdn_scan_bwd_workspace_bytes(BH, N, dh, 1, ns) == 4 * (2 * nseg * per + 2 * BH * dh * dh)
    assert lib.gmdn_scan_bwd_workspace_bytes(BH, N, dh, 1, ns) <= 1024 << 20
    p = [0x1000] * 16
    # adam / muon without workspace -> GMDN_ERR_WORKSPACE
    assert lib.gmdn_scan_bwd(*p, None, 0, 4, 16, 64, 2, 3, 0, None) == 3
    assert lib.gmdn_scan_bwd(*p, None, 0, 4, 16, 64, 1, 3, 0, None) == 3


def test_chunk_desc_layout_matches_header():
    # 3 int64 + 6 int32 + float + pad + 12 int64
    assert ctypes.sizeof(_native.ChunkDesc) == 3 * 8 + 6 * 4 + 4 + 4 + 12 * 8


def test_front_argument_checks():
    lib = _native.load()
    p = 0x1000
    # y, weight, bias, q, k, v, B, T, D, dh, K, dtype, stream
    assert lib.gmdn_front_fwd(p, p, p, p, p, p, 2, 64, 256, 96, 4, 0, None) == 2   # dh not built
    assert lib.gmdn_front_fwd(p, p, p, p, p, p, 2, 64, 200, 128, 4, 0, None) == 1  # D not a multiple of dh
    assert lib.gmdn_front_fwd(p, p, p, p, p, p, 2, 64, 256, 128, 5, 0, None) == 1  # kernel above 4
    assert lib.gmdn_front_fwd(p, p, p, p, p, p, 2, 64, 256, 128, 4, 7, None) == 2  # dtype
    assert lib.gmdn_front_fwd(None, p, p, p, p, p, 2, 64, 256, 128, 4, 0, None) == 1
    assert lib.gmdn_front_fwd(p + 2, p, p, p, p, p, 2, 64, 256, 128, 4, 0, None) == 1  # misaligned y
    assert lib.gmdn_front_fwd(None, None, None, None, None, None, 0, 64, 256, 128, 4, 0, None) == 0  # empty
    assert lib.gmdn_front_bwd(p, p, p, p, p, p, p, None, 2, 64, 256, 128, 4, 0, None) == 1  # no workspace
    assert lib.gmdn_front_bwd_workspace_floats(2, 65, 256, 4) == 2 * 2 * 768 * 5


def test_msign_workspace_and_argument_validation():
    lib = _native.load()
    assert lib.gmdn_msign_workspace_bytes(0, 4, 4) == 0
    assert lib.gmdn_msign_workspace_bytes(1, 0, 4) == 0
    assert lib.gmdn_msign_workspace_bytes(1, 40000, 4) == 0
    # 24 x 1024 pads to 128 x 1024: two X buffers, A and Bm (128 x 128), 64 partial sums, 256-aligned
    x, a = 128 * 1024 * 4, 128 * 128 * 4
    assert lib.gmdn_msign_workspace_bytes(1, 24, 1024) == 2 * x + 2 * a + 256
    assert lib.gmdn_msign_workspace_bytes(3, 1024, 24) == 2 * 3 * x + 2 * 3 * a + 768
    p = 0x1000

    def call(M=p, out=p, batch=2, rows=8, cols=8, steps=5, eps=1e-7, dtype=1, ws=0x100000, wsb=1 << 30):
        return lib.gmdn_msign(M, out, batch, rows, cols, steps, eps, dtype, ws, wsb, None)

    assert call(batch=-1) == 1 and call(batch=65536) == 1
    assert call(steps=-1) == 1 and call(steps=65) == 1
    assert call(eps=float("nan")) == 1 and call(eps=-1.0) == 1
    assert call(dtype=7) == 2
    assert call(rows=40000) == 2
    assert call(M=None) == 1 and call(out=None) == 1
    assert call(ws=None) == 3
    assert call(wsb=16) == 3
    assert call(ws=0x100010) == 3  # workspace not 256-byte aligned
    assert call(batch=0) == 0 and call(rows=0) == 0  # empty: nothing to do, nothing launched


def _chunk_desc(rule=0, d=64, T=128, so=None):
    desc = _native.ChunkDesc()
    desc.B, desc.H, desc.T, desc.d, desc.C = 1, 2, T, d, 64
    desc.rule, desc.ns, desc.dtype, desc.eps = rule, 3, _native.DTYPE_BF16, 1e-6
    st = (2 * T * d, T * d, d)
    for name in ("sq", "sk", "sv", "so"):
        arr = getattr(desc, name)
        for i in range(3):
            arr[i] = (so if (name == "so" and so is not None) else st)[i]
    return desc


def test_chunk_bwd_rejects_misaligned_streams():
    """dO tiles are LDS-DMA loads planned from its strides, dq and dk leave in
    16-byte pieces: unaligned strides or pointers are refused with
    GMDN_ERR_UNSUPPORTED before anything is launched."""
    lib = _native.load()
    p, ws = 0x1000, 0x100000

    def call(desc, dq=p, dk=p, dv=p, dO=p):
        need = lib.gmdn_chunk_bwd_workspace_bytes(desc)
        return lib.gmdn_chunk_bwd(desc, p, p, p, p, p, None, None, p, dO, dq, dk, dv, p, p, None, None, ws,
                                  need, None)

    good = _chunk_desc()
    assert lib.gmdn_chunk_bwd_workspace_bytes(good) > 0
    assert call(_chunk_desc(so=(2 * 128 * 64, 128 * 64, 68))) == 2   # dO token stride not 8 elements
    assert call(_chunk_desc(so=(2 * 128 * 64 + 4, 128 * 64, 64))) == 2  # dO batch stride
    assert call(good, dq=p + 2) == 2
    assert call(good, dk=p + 8) == 2
    assert call(good, dv=p + 4) == 2
    assert call(good, dO=p + 2) == 2


def test_chunk_bwd_muon_workspace_floor():
    """The fused muon backward in 'tf32' runs with any workspace down to
    one-chunk segments of its reverse scan (its prefix -- Kw, Uv, gS, dU per
    chunk and the chunk scalars and their gradients, 256-byte aligned -- plus
    one chunk's iterates, |M_i| and the carried Mbar, Sb per (b, h)); below
    that it is refused with GMDN_ERR_WORKSPACE before anything is launched,
    and in 'ieee' below the default size."""
    lib = _native.load()
    p = 0x1000
    B, H, T, d, ns = 1, 2, 448, 64, 3
    desc = _chunk_desc(rule=1, d=d, T=T)
    desc.precision = _native.PREC_TF32
    BH, N, mat = B * H, T // 64, d * d
    BHN = BH * N
    prefix = (4 * BHN * mat + 8 * BHN + 63) // 64 * 64
    floor = 4 * (prefix + BH * ((3 * ns + 2) * mat + 1) + 2 * BH * mat)
    full = lib.gmdn_chunk_bwd_workspace_bytes(desc)
    assert full > floor

    def call(nbytes):
        return lib.gmdn_chunk_bwd(desc, p, p, p, p, p, p, None, p, p, p, p, p, p, p, p, None, p, nbytes, None)

    assert call(floor - 4) == 3
    desc.precision = _native.PREC_IEEE
    assert call(full - 4) == 3
