"""C ABI of libmxgg.so without a GPU: it loads, exports every function that
include/mxgg.h declares, and rejects bad arguments before touching the device.

Every call below fails validation on the host (null pointers, bad shapes,
misalignment, unknown enums), so no kernel is launched.
"""
import ctypes
import re
from pathlib import Path

import pytest

from mxfp8gg import _lib

ROOT = Path(__file__).resolve().parent.parent
HEADER = ROOT / "include" / "mxgg.h"


def declared_functions():
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(mxgg_\w+)\s*\(", text)))


@pytest.fixture(scope="module")
def lib():
    return _lib.load()


def test_header_lists_the_bound_functions():
    assert declared_functions() == sorted(_lib.SIGNATURES)


def _ctype_of(decl: str):
    """ctypes type of one C parameter or return type of the header (every
    scalar there is int or int64_t, every pointer T*)."""
    decl = decl.strip()
    if decl == "const char*":
        return ctypes.c_char_p
    if "*" in decl:
        return ctypes.c_void_p
    kind = decl.split()[0]
    return {"int64_t": ctypes.c_int64, "int": ctypes.c_int}[kind]


def test_bound_signatures_match_the_header():
    """Every argument of every binding has the width and kind the header
    declares, so no call passes a 32-bit value where the library reads 64."""
    text = re.sub(r"/\*.*?\*/|//[^\n]*", "", HEADER.read_text(), flags=re.S)
    decls = re.findall(r"([A-Za-z_][\w ]*\*?)\s*\b(mxgg_\w+)\s*\(([^)]*)\)\s*;", text)
    assert sorted(name for _, name, _ in decls) == sorted(_lib.SIGNATURES)
    for ret, name, params in decls:
        params = " ".join(params.split())
        want = [] if params in ("", "void") else [_ctype_of(p.rsplit(" ", 1)[0])
                                                  for p in params.split(",")]
        res, args = _lib.SIGNATURES[name]
        assert res is _ctype_of(ret.replace(" *", "*")), name
        assert list(args) == want, name


def test_integration_stubs_match_the_bindings():
    """The ctypes stubs of the integration guide at the repository root (what a
    maintainer would copy into the reference's code) declare the argument and
    return types mxfp8gg binds, and assert the header's ABI version."""
    import ast
    text = (ROOT / "INTEGRATION.md").read_text()
    blocks = re.findall(r"```python\n(.*?)```", text, flags=re.S)
    ns = {"ctypes": ctypes, "P": ctypes.c_void_p, "I64": ctypes.c_int64, "I": ctypes.c_int}

    class Fn:
        argtypes = None
        restype = None

    fns = {}

    class Lib:
        def __getattr__(self, name):
            return fns.setdefault(name, Fn())

    ns["_lib"] = Lib()
    version = int(re.search(r"#define MXGG_ABI_VERSION (\d+)", HEADER.read_text()).group(1))
    checked = asserted = 0
    for block in blocks:
        for node in ast.walk(ast.parse(block)):
            if isinstance(node, ast.Assign) and isinstance(node.targets[0], ast.Attribute):
                tgt = node.targets[0]
                if (tgt.attr in ("argtypes", "restype") and isinstance(tgt.value, ast.Attribute)
                        and isinstance(tgt.value.value, ast.Name) and tgt.value.value.id == "_lib"):
                    name = tgt.value.attr
                    value = eval(compile(ast.Expression(node.value), "stub", "eval"), ns)
                    setattr(fns.setdefault(name, Fn()), tgt.attr, value)
                    res, args = _lib.SIGNATURES[name]
                    assert value == (list(args) if tgt.attr == "argtypes" else res), name
                    checked += 1
            if isinstance(node, ast.Assert) and "mxgg_abi_version" in ast.unparse(node):
                assert node.test.comparators[0].value == version
                asserted += 1
    assert checked >= 6 and asserted == 1


def test_library_exports_every_declared_symbol(lib):
    for name in declared_functions():
        assert hasattr(lib, name), name


def test_abi_version_and_status_strings(lib):
    assert lib.mxgg_abi_version() == _lib.ABI_VERSION
    for code in range(0, 7):
        assert lib.mxgg_status_string(code)
    assert lib.mxgg_status_string(99) == b"unknown status"


FAKE = 0x10000  # 16-byte aligned, never dereferenced: validation fails first


def _fwd(lib, **kw):
    args = dict(a=FAKE, lda=256, a_s=None, ldas=0, w=FAKE, wg=512 * 256, ldw=256, w_s=None,
                wsg=0, ldws=0, ends=None, E=1, M=64, N=512, K=256, out=FAKE, ldo=512,
                dt=_lib.OUT_BF16)
    args.update(kw)
    return lib.mxgg_grouped_fwd(args["a"], args["lda"], args["a_s"], args["ldas"], args["w"],
                                args["wg"], args["ldw"], args["w_s"], args["wsg"], args["ldws"],
                                args["ends"], args["E"], args["M"], args["N"], args["K"],
                                args["out"], args["ldo"], args["dt"], None)


def _fwd_split(lib, ws=FAKE, nbytes=None, **kw):
    args = dict(a=FAKE, lda=256, a_s=None, ldas=0, w=FAKE, wg=512 * 256, ldw=256, w_s=None,
                wsg=0, ldws=0, ends=None, E=1, M=64, N=512, K=256, out=FAKE, ldo=512,
                dt=_lib.OUT_BF16)
    args.update(kw)
    if nbytes is None:
        nbytes = lib.mxgg_grouped_fwd_workspace_bytes()
    return lib.mxgg_grouped_fwd_split(args["a"], args["lda"], args["a_s"], args["ldas"],
                                      args["w"], args["wg"], args["ldw"], args["w_s"],
                                      args["wsg"], args["ldws"], args["ends"], args["E"],
                                      args["M"], args["N"], args["K"], args["out"], args["ldo"],
                                      args["dt"], ws, nbytes, None)


def test_wgrad_split_workspace_bound(lib):
    # header + one 256x256 fp32 partial per work item, with at most
    # M / split + E chunks over all experts; -1 for invalid arguments
    assert lib.mxgg_grouped_wgrad_workspace_bytes(65536, 1024, 1024, 2, 4096) == \
        32768 + (16 + 2) * 16 * 256 * 256 * 4
    assert lib.mxgg_grouped_wgrad_workspace_bytes(65536, 1024, 1024, 2, 0) == -1
    assert lib.mxgg_grouped_wgrad_workspace_bytes(65536, 1024, 1024, 0, 4096) == -1


@pytest.mark.parametrize("kw,status", [
    (dict(split=0), _lib.ERR_INVALID_ARGUMENT),
    (dict(split=200), _lib.ERR_INVALID_ARGUMENT),
    (dict(ws=None), _lib.ERR_INVALID_ARGUMENT),
    (dict(nbytes=32768), _lib.ERR_SHAPE),
    (dict(ws=FAKE + 4), _lib.ERR_ALIGNMENT),
    (dict(M=100), _lib.ERR_SHAPE),                     # then the wgrad's own checks
])
def test_grouped_wgrad_split_rejects(lib, kw, status):
    a = dict(go=FAKE, ldgo=4096, gs=None, ldgs=0, ia=FAKE, ldia=4096, is_=None, ldis=0,
             ends=FAKE, E=2, M=4096, N=256, K=256, dw=FAKE, dt=_lib.OUT_F32, split=1024,
             ws=FAKE, nbytes=None)
    a.update(kw)
    if a["nbytes"] is None:
        a["nbytes"] = max(0, lib.mxgg_grouped_wgrad_workspace_bytes(a["M"], a["N"], a["K"],
                                                                    a["E"], 1024))
    assert lib.mxgg_grouped_wgrad_split(a["go"], a["ldgo"], a["gs"], a["ldgs"], a["ia"],
                                        a["ldia"], a["is_"], a["ldis"], a["ends"], a["E"],
                                        a["M"], a["N"], a["K"], a["dw"], a["dt"], a["split"],
                                        a["ws"], a["nbytes"], None) == status


def test_split_workspace_size_covers_one_partial_per_unit(lib):
    # header + one 256x256 fp32 partial per workgroup of the persistent grid
    n = lib.mxgg_grouped_fwd_workspace_bytes()
    assert n >= 16384 + 8 * 256 * 256 * 4 and (n - 16384) % (256 * 256 * 4) == 0


@pytest.mark.parametrize("kw,status", [
    (dict(ws=None), _lib.ERR_INVALID_ARGUMENT),
    (dict(nbytes=16384), _lib.ERR_SHAPE),
    (dict(ws=FAKE + 8), _lib.ERR_ALIGNMENT),
    (dict(K=100), _lib.ERR_SHAPE),                     # then the forward's own checks
    (dict(a=None), _lib.ERR_INVALID_ARGUMENT),
])
def test_grouped_fwd_split_rejects(lib, kw, status):
    assert _fwd_split(lib, **kw) == status


@pytest.mark.parametrize("kw,status", [
    (dict(K=100), _lib.ERR_SHAPE),                     # K % 32
    (dict(K=0), _lib.ERR_SHAPE),
    (dict(M=-1), _lib.ERR_SHAPE),
    (dict(dt=7), _lib.ERR_INVALID_ARGUMENT),
    (dict(a_s=FAKE, ldas=8), _lib.ERR_INVALID_ARGUMENT),  # only one of the scales
    (dict(a=None), _lib.ERR_INVALID_ARGUMENT),
    (dict(lda=128), _lib.ERR_SHAPE),                   # ld < K
    (dict(a=FAKE + 8), _lib.ERR_ALIGNMENT),
    (dict(lda=264), _lib.ERR_ALIGNMENT),               # not a multiple of 16
    (dict(out=FAKE + 2), _lib.ERR_ALIGNMENT),
    (dict(ends=FAKE, E=0), _lib.ERR_UNSUPPORTED),
    (dict(ends=FAKE, E=2000), _lib.ERR_UNSUPPORTED),
    (dict(ends=FAKE, E=4, wg=-16), _lib.ERR_SHAPE),    # negative expert stride
    (dict(ends=FAKE, E=4, wg=100), _lib.ERR_ALIGNMENT),  # expert stride not a multiple of 16
    (dict(a_s=FAKE, ldas=32, w_s=FAKE, ldws=512, wsg=512 * 8), _lib.ERR_SHAPE),  # ldas < M
    (dict(a_s=FAKE, ldas=66, w_s=FAKE, ldws=512, wsg=512 * 8), _lib.ERR_ALIGNMENT),
    (dict(a_s=FAKE + 2, ldas=64, w_s=FAKE, ldws=512, wsg=512 * 8), _lib.ERR_ALIGNMENT),
    (dict(a_s=FAKE, ldas=64, w_s=FAKE, ldws=512, wsg=-4, ends=FAKE, E=4), _lib.ERR_SHAPE),
    (dict(a_s=FAKE, ldas=64, w_s=FAKE, ldws=512, wsg=102, ends=FAKE, E=4), _lib.ERR_ALIGNMENT),
])
def test_grouped_fwd_rejects(lib, kw, status):
    assert _fwd(lib, **kw) == status
    assert lib.mxgg_last_error()


def test_grouped_fwd_empty_is_noop(lib):
    assert _fwd(lib, M=0, a=None, w=None, out=None) == _lib.OK


def _wg(lib, **kw):
    args = dict(go=FAKE, ldgo=128, gs=None, ldgs=0, ia=FAKE, ldia=128, is_=None, ldis=0,
                ends=FAKE, E=4, M=128, N=64, K=64, dw=FAKE, dt=_lib.OUT_F32, split=0)
    args.update(kw)
    return lib.mxgg_grouped_wgrad(args["go"], args["ldgo"], args["gs"], args["ldgs"], args["ia"],
                                  args["ldia"], args["is_"], args["ldis"], args["ends"], args["E"],
                                  args["M"], args["N"], args["K"], args["dw"], args["dt"],
                                  args["split"], None)


@pytest.mark.parametrize("kw,status", [
    (dict(M=100), _lib.ERR_SHAPE),                     # tokens % 32
    (dict(ends=None), _lib.ERR_INVALID_ARGUMENT),
    (dict(E=0), _lib.ERR_UNSUPPORTED),
    (dict(gs=FAKE, ldgs=4), _lib.ERR_INVALID_ARGUMENT),
    (dict(dw=None), _lib.ERR_INVALID_ARGUMENT),
    (dict(ldgo=64), _lib.ERR_SHAPE),
    (dict(go=FAKE + 4), _lib.ERR_ALIGNMENT),
    (dict(K=66), _lib.ERR_ALIGNMENT),
    (dict(dt=3), _lib.ERR_INVALID_ARGUMENT),
    (dict(gs=FAKE, ldgs=32, is_=FAKE, ldis=64), _lib.ERR_SHAPE),     # ldgos < N
    (dict(gs=FAKE, ldgs=66, is_=FAKE, ldis=64), _lib.ERR_ALIGNMENT),
    (dict(split=100), _lib.ERR_INVALID_ARGUMENT),      # split-K chunk % 128
    (dict(split=-128), _lib.ERR_INVALID_ARGUMENT),
    (dict(split=256, dt=_lib.OUT_BF16), _lib.ERR_UNSUPPORTED),  # atomics need fp32
])
def test_grouped_wgrad_rejects(lib, kw, status):
    assert _wg(lib, **kw) == status


RM, BM = _lib.SCALES_ROW_MAJOR, _lib.SCALES_BLOCK_MAJOR


@pytest.mark.parametrize("args,status", [
    ((FAKE, 4, 100, 100, FAKE, 100, FAKE, 4, RM, 0, None), _lib.ERR_SHAPE),      # cols % 32
    ((FAKE, 4, 64, 64, FAKE, 64, FAKE, 2, RM, 5, None), _lib.ERR_INVALID_ARGUMENT),  # mode
    ((FAKE, 4, 64, 64, FAKE, 64, FAKE, 2, 7, 0, None), _lib.ERR_INVALID_ARGUMENT),  # layout
    ((None, 4, 64, 64, FAKE, 64, FAKE, 2, RM, 0, None), _lib.ERR_INVALID_ARGUMENT),
    ((FAKE + 2, 4, 64, 64, FAKE, 64, FAKE, 2, RM, 0, None), _lib.ERR_ALIGNMENT),
    ((FAKE, 4, 64, 32, FAKE, 64, FAKE, 2, RM, 0, None), _lib.ERR_SHAPE),       # ldx < cols
    ((FAKE, 40, 64, 64, FAKE, 64, FAKE, 32, BM, 0, None), _lib.ERR_SHAPE),     # block ld < rows
])
def test_quant_dim0_rejects(lib, args, status):
    assert lib.mxgg_quant_dim0(*args) == status


def test_quant_dim0_empty_is_noop(lib):
    assert lib.mxgg_quant_dim0(None, 0, 64, 64, None, 64, None, 2, RM, 0, None) == _lib.OK


@pytest.mark.parametrize("args,status", [
    ((FAKE, 1, -1, 4, 0, 4, FAKE, 0, 16), _lib.ERR_SHAPE),
    ((None, 1, 8, 4, 0, 4, FAKE, 0, 16), _lib.ERR_INVALID_ARGUMENT),
    ((FAKE, 1, 8, 4, 0, 2, FAKE, 0, 16), _lib.ERR_SHAPE),           # lds < nblk
    ((FAKE, 1, 20, 4, 0, 4, FAKE, 0, 16), _lib.ERR_SHAPE),          # ldd < rows
    ((FAKE, 2, 8, 4, 16, 4, FAKE, 64, 16), _lib.ERR_SHAPE),         # src batch stride
    ((FAKE, 70000, 8, 4, 32, 4, FAKE, 64, 16), _lib.ERR_UNSUPPORTED),
])
def test_scales_to_block_major_rejects(lib, args, status):
    assert lib.mxgg_scales_to_block_major(*args, None) == status


def test_scales_to_block_major_empty_is_noop(lib):
    assert lib.mxgg_scales_to_block_major(None, 0, 8, 4, 0, 4, None, 0, 16, None) == _lib.OK


@pytest.mark.parametrize("kw,status", [
    (dict(cols=12), _lib.ERR_SHAPE),
    (dict(cap=48), _lib.ERR_SHAPE),                    # not a multiple of 32
    (dict(cap=32), _lib.ERR_SHAPE),                    # below rows + 31 * groups
    (dict(E=0), _lib.ERR_UNSUPPORTED),
    (dict(pad=None), _lib.ERR_INVALID_ARGUMENT),
    (dict(mode=9), _lib.ERR_INVALID_ARGUMENT),
    (dict(x=FAKE + 2), _lib.ERR_ALIGNMENT),
    (dict(layout=3), _lib.ERR_INVALID_ARGUMENT),
    (dict(layout=BM, ldst=32), _lib.ERR_SHAPE),        # block ld < cols
])
def test_quant_dim1_rejects(lib, kw, status):
    a = dict(x=FAKE, rows=64, cols=64, ldx=64, ends=FAKE, E=2, cap=128, qt=FAKE, ldqt=128,
             st=FAKE, ldst=4, layout=RM, pad=FAKE, mode=0)
    a.update(kw)
    assert lib.mxgg_quant_dim1(a["x"], a["rows"], a["cols"], a["ldx"], a["ends"], a["E"],
                               a["cap"], a["qt"], a["ldqt"], a["st"], a["ldst"], a["layout"],
                               a["pad"], a["mode"], None) == status


def _dual(lib, **kw):
    a = dict(x=FAKE, rows=64, cols=64, ldx=64, ends=FAKE, E=2, cap=128, q=FAKE, ldq=64, s=FAKE,
             lds=64, qt=FAKE, ldqt=128, st=FAKE, ldst=64, layout=BM, pad=FAKE, mode=0)
    a.update(kw)
    return lib.mxgg_quant_dual(a["x"], a["rows"], a["cols"], a["ldx"], a["ends"], a["E"],
                               a["cap"], a["q"], a["ldq"], a["s"], a["lds"], a["qt"], a["ldqt"],
                               a["st"], a["ldst"], a["layout"], a["pad"], a["mode"], None)


@pytest.mark.parametrize("kw,status", [
    (dict(cols=40), _lib.ERR_SHAPE),                 # the row-wise cast needs cols % 32
    (dict(cap=64), _lib.ERR_SHAPE),                  # below rows + 31 * groups
    (dict(cap=100), _lib.ERR_SHAPE),
    (dict(E=0), _lib.ERR_UNSUPPORTED),
    (dict(pad=None), _lib.ERR_INVALID_ARGUMENT),
    (dict(q=None), _lib.ERR_INVALID_ARGUMENT),
    (dict(qt=None), _lib.ERR_INVALID_ARGUMENT),
    (dict(mode=3), _lib.ERR_INVALID_ARGUMENT),
    (dict(layout=5), _lib.ERR_INVALID_ARGUMENT),
    (dict(lds=32), _lib.ERR_SHAPE),                  # block-major ld < rows
    (dict(ldst=32), _lib.ERR_SHAPE),                 # block-major ld < cols
    (dict(x=FAKE + 8), _lib.ERR_ALIGNMENT),
    (dict(q=FAKE + 4), _lib.ERR_ALIGNMENT),
    (dict(ldqt=136), _lib.ERR_ALIGNMENT),
])
def test_quant_dual_rejects(lib, kw, status):
    assert _dual(lib, **kw) == status


def test_quant_dual_empty_is_noop(lib):
    assert _dual(lib, cols=0) == _lib.OK


def _swiglu0(lib, **kw):
    a = dict(g=FAKE, u=FAKE + 128, ldh=128, rows=8, cols=64, aout=None, lda=64, q=FAKE, ldq=64,
             s=FAKE, lds=8, layout=BM, mode=0)
    a.update(kw)
    return lib.mxgg_swiglu_quant_dim0(a["g"], a["u"], a["ldh"], a["rows"], a["cols"], a["aout"],
                                      a["lda"], a["q"], a["ldq"], a["s"], a["lds"], a["layout"],
                                      a["mode"], None)


@pytest.mark.parametrize("kw,status", [
    (dict(cols=48), _lib.ERR_SHAPE),
    (dict(rows=-1), _lib.ERR_SHAPE),
    (dict(mode=4), _lib.ERR_INVALID_ARGUMENT),
    (dict(layout=2), _lib.ERR_INVALID_ARGUMENT),
    (dict(u=None), _lib.ERR_INVALID_ARGUMENT),
    (dict(ldh=32), _lib.ERR_SHAPE),                  # ldh < cols
    (dict(lds=4), _lib.ERR_SHAPE),                   # block-major ld < rows
    (dict(u=FAKE + 8), _lib.ERR_ALIGNMENT),
    (dict(ldh=132), _lib.ERR_ALIGNMENT),
    (dict(aout=FAKE, lda=68), _lib.ERR_ALIGNMENT),
])
def test_swiglu_quant_dim0_rejects(lib, kw, status):
    assert _swiglu0(lib, **kw) == status


def test_swiglu_quant_dim0_empty_is_noop(lib):
    assert _swiglu0(lib, rows=0, g=None, u=None, q=None, s=None) == _lib.OK


def _fwd_swiglu(lib, keep_h, **kw):
    a = dict(a=FAKE, lda=256, a_s=None, ldas=0, w=FAKE, wg=512 * 256, ldw=256, w_s=None, wsg=0,
             ldws=0, ends=None, E=1, M=64, F=256, K=256, h=FAKE, ldh=512, q=FAKE, ldq=256,
             s=FAKE, lds=64, layout=BM, mode=0)
    a.update(kw)
    head = (a["a"], a["lda"], a["a_s"], a["ldas"], a["w"], a["wg"], a["ldw"], a["w_s"], a["wsg"],
            a["ldws"], a["ends"], a["E"], a["M"], a["F"], a["K"])
    tail = (a["q"], a["ldq"], a["s"], a["lds"], a["layout"], a["mode"], None)
    if keep_h:
        return lib.mxgg_grouped_fwd_swiglu_quant_keep_h(*head, a["h"], a["ldh"], *tail)
    return lib.mxgg_grouped_fwd_swiglu_quant(*head, *tail)


@pytest.mark.parametrize("keep_h", [False, True])
@pytest.mark.parametrize("kw,status", [
    (dict(mode=4), _lib.ERR_INVALID_ARGUMENT),
    (dict(layout=2), _lib.ERR_INVALID_ARGUMENT),
    (dict(F=192), _lib.ERR_SHAPE),                   # F % 128 != 0
    (dict(q=None), _lib.ERR_INVALID_ARGUMENT),
    (dict(ldq=128), _lib.ERR_SHAPE),                 # ldq < F
    (dict(lds=32), _lib.ERR_SHAPE),                  # block-major ld < M
    (dict(q=FAKE + 4), _lib.ERR_ALIGNMENT),
    (dict(K=100), _lib.ERR_SHAPE),
    (dict(a=None), _lib.ERR_INVALID_ARGUMENT),
])
def test_grouped_fwd_swiglu_quant_rejects(lib, keep_h, kw, status):
    assert _fwd_swiglu(lib, keep_h, **kw) == status


@pytest.mark.parametrize("kw,status", [
    (dict(h=None), _lib.ERR_INVALID_ARGUMENT),
    (dict(ldh=384), _lib.ERR_SHAPE),                 # ldh < 2F
    (dict(h=FAKE + 8), _lib.ERR_ALIGNMENT),
    (dict(ldh=516), _lib.ERR_ALIGNMENT),             # ldh % 8 != 0
])
def test_grouped_fwd_swiglu_quant_keep_h_rejects(lib, kw, status):
    assert _fwd_swiglu(lib, True, **kw) == status


def test_grouped_fwd_swiglu_quant_empty_is_noop(lib):
    for keep_h in (False, True):
        assert _fwd_swiglu(lib, keep_h, M=0, a=None, h=None, q=None, s=None) == _lib.OK


def _swiglu_bwd(lib, **kw):
    a = dict(g=FAKE, u=FAKE + 128, ldh=128, da=FAKE, ldga=64, rows=64, cols=64, ends=FAKE, E=2,
             cap=128, dq=FAKE, lddq=128, ds=FAKE, ldds=64, dqt=FAKE, lddqt=128, dst=FAKE,
             lddst=128, aqt=FAKE, ldaqt=128, ast=FAKE, ldast=64, pad=FAKE, dh=None, lddh=128,
             layout=BM, mode=0)
    a.update(kw)
    return lib.mxgg_swiglu_bwd_quant(
        a["g"], a["u"], a["ldh"], a["da"], a["ldga"], a["rows"], a["cols"], a["ends"], a["E"],
        a["cap"], a["dq"], a["lddq"], a["ds"], a["ldds"], a["dqt"], a["lddqt"], a["dst"],
        a["lddst"], a["aqt"], a["ldaqt"], a["ast"], a["ldast"], a["pad"], a["dh"], a["lddh"],
        a["layout"], a["mode"], None)


@pytest.mark.parametrize("kw,status", [
    (dict(cols=40), _lib.ERR_SHAPE),
    (dict(cap=96), _lib.ERR_SHAPE),                  # below rows + 31 * groups
    (dict(cap=120), _lib.ERR_SHAPE),                 # not a multiple of 32
    (dict(E=0), _lib.ERR_UNSUPPORTED),
    (dict(E=1025), _lib.ERR_UNSUPPORTED),
    (dict(pad=None), _lib.ERR_INVALID_ARGUMENT),
    (dict(da=None), _lib.ERR_INVALID_ARGUMENT),
    (dict(aqt=None), _lib.ERR_INVALID_ARGUMENT),
    (dict(mode=7), _lib.ERR_INVALID_ARGUMENT),
    (dict(lddq=64), _lib.ERR_SHAPE),                 # dh row is 2 * cols wide
    (dict(lddst=64), _lib.ERR_SHAPE),                # block-major ld < 2 * cols
    (dict(ldast=32), _lib.ERR_SHAPE),
    (dict(da=FAKE + 4), _lib.ERR_ALIGNMENT),
    (dict(lddqt=136), _lib.ERR_ALIGNMENT),
    (dict(dq=FAKE + 4), _lib.ERR_ALIGNMENT),
    (dict(dh=FAKE + 8), _lib.ERR_ALIGNMENT),
    # 1024 position blocks x 16384 feature blocks of 128: 2^24 workgroups, over the grid limit
    (dict(cols=1 << 21, ldh=2 << 21, ldga=1 << 21, lddq=2 << 21, cap=131072, lddqt=131072,
          ldaqt=131072, lddst=2 << 21, ldast=1 << 21), _lib.ERR_UNSUPPORTED),
])
def test_swiglu_bwd_quant_rejects(lib, kw, status):
    assert _swiglu_bwd(lib, **kw) == status


def test_swiglu_bwd_quant_empty_is_noop(lib):
    assert _swiglu_bwd(lib, cols=0) == _lib.OK


def test_python_maps_errors_to_exceptions(lib):
    with pytest.raises(ValueError, match="K=100"):
        _lib.check(_fwd(lib, K=100), "grouped_fwd")


# ---------------------------------------------------------------------------
# Token routing entry points
# ---------------------------------------------------------------------------
def _route(lib, **kw):
    a = dict(idx=FAKE, T=64, K=2, E=4, pad=32, cap=128 + 4 * 31, perm=FAKE, src=FAKE, ends=FAKE,
             counts=FAKE)
    a.update(kw)
    return lib.mxgg_route_plan(a["idx"], a["T"], a["K"], a["E"], a["pad"], a["cap"], a["perm"],
                               a["src"], a["ends"], a["counts"], None)


@pytest.mark.parametrize("kw,status", [
    (dict(E=0), _lib.ERR_UNSUPPORTED),
    (dict(E=1025), _lib.ERR_UNSUPPORTED),
    (dict(pad=0), _lib.ERR_UNSUPPORTED),
    (dict(pad=2048), _lib.ERR_UNSUPPORTED),
    (dict(K=0), _lib.ERR_SHAPE),
    (dict(T=-1), _lib.ERR_SHAPE),
    (dict(cap=128 + 4 * 31 - 1), _lib.ERR_SHAPE),      # below tokens*topk + E*(pad-1)
    (dict(T=1 << 30, K=4, cap=1 << 31), _lib.ERR_UNSUPPORTED),
    (dict(ends=None), _lib.ERR_INVALID_ARGUMENT),
    (dict(src=None), _lib.ERR_INVALID_ARGUMENT),
    (dict(idx=None), _lib.ERR_INVALID_ARGUMENT),
])
def test_route_plan_rejects(lib, kw, status):
    assert _route(lib, **kw) == status


def test_route_plan_workspace_size(lib):
    # one int32 count per (workgroup of 4096 slots, expert); -1 when invalid
    assert lib.mxgg_route_plan_workspace_bytes(16384, 8, 32) == 32 * 32 * 4
    assert lib.mxgg_route_plan_workspace_bytes(4097, 1, 3) == 2 * 3 * 4
    assert lib.mxgg_route_plan_workspace_bytes(0, 2, 4) == 0
    assert lib.mxgg_route_plan_workspace_bytes(64, 0, 4) == -1
    assert lib.mxgg_route_plan_workspace_bytes(64, 2, 1025) == -1


@pytest.mark.parametrize("kw,status", [
    (dict(E=0), _lib.ERR_UNSUPPORTED),                  # the shared checks come first
    (dict(ws=None), _lib.ERR_INVALID_ARGUMENT),
    (dict(ws=FAKE + 2), _lib.ERR_ALIGNMENT),
    (dict(nbytes=4), _lib.ERR_SHAPE),                   # 64 * 2 slots, 4 experts: 16 bytes
])
def test_route_plan_ws_rejects(lib, kw, status):
    a = dict(idx=FAKE, T=64, K=2, E=4, pad=32, cap=128 + 4 * 31, perm=FAKE, src=FAKE, ends=FAKE,
             counts=FAKE, ws=FAKE, nbytes=16)
    a.update(kw)
    assert lib.mxgg_route_plan_ws(a["idx"], a["T"], a["K"], a["E"], a["pad"], a["cap"], a["perm"],
                                  a["src"], a["ends"], a["counts"], a["ws"], a["nbytes"],
                                  None) == status


def _gather(lib, **kw):
    a = dict(x=FAKE, T=16, cols=64, ldx=64, src=FAKE, K=2, scale=None, rows=40, out=FAKE, ldo=64)
    a.update(kw)
    return lib.mxgg_gather_rows(a["x"], a["T"], a["cols"], a["ldx"], a["src"], a["K"], a["scale"],
                                a["rows"], a["out"], a["ldo"], None)


@pytest.mark.parametrize("kw,status", [
    (dict(cols=60), _lib.ERR_SHAPE),
    (dict(ldo=56), _lib.ERR_SHAPE),
    (dict(K=0), _lib.ERR_SHAPE),
    (dict(x=FAKE + 8), _lib.ERR_ALIGNMENT),
    (dict(ldx=72 + 4), _lib.ERR_ALIGNMENT),
    (dict(src=None), _lib.ERR_INVALID_ARGUMENT),
    (dict(rows=1 << 27), _lib.ERR_UNSUPPORTED),
])
def test_gather_rows_rejects(lib, kw, status):
    assert _gather(lib, **kw) == status


def test_gather_rows_empty_is_noop(lib):
    assert _gather(lib, rows=0) == _lib.OK


def _gather_dual(lib, **kw):
    a = dict(x=FAKE, T=32, cols=64, ldx=64, src=FAKE, K=2, scale=None, rows=64, ends=FAKE, E=2,
             cap=128, q=FAKE, ldq=64, s=FAKE, lds=64, qt=FAKE, ldqt=128, st=FAKE, ldst=64,
             layout=BM, pad=FAKE, mode=0)
    a.update(kw)
    return lib.mxgg_gather_quant_dual(
        a["x"], a["T"], a["cols"], a["ldx"], a["src"], a["K"], a["scale"], a["rows"], a["ends"],
        a["E"], a["cap"], a["q"], a["ldq"], a["s"], a["lds"], a["qt"], a["ldqt"], a["st"],
        a["ldst"], a["layout"], a["pad"], a["mode"], None)


@pytest.mark.parametrize("kw,status", [
    (dict(K=0), _lib.ERR_SHAPE),
    (dict(cols=48), _lib.ERR_SHAPE),
    (dict(cap=96), _lib.ERR_SHAPE),                   # below rows + 31 * groups
    (dict(src=None), _lib.ERR_INVALID_ARGUMENT),
    (dict(mode=9), _lib.ERR_INVALID_ARGUMENT),
    (dict(x=FAKE + 4), _lib.ERR_ALIGNMENT),
    (dict(E=0), _lib.ERR_UNSUPPORTED),
])
def test_gather_quant_dual_rejects(lib, kw, status):
    assert _gather_dual(lib, **kw) == status


def _gather_dim0(lib, **kw):
    a = dict(x=FAKE, T=32, cols=64, ldx=64, src=FAKE, K=2, rows=64, q=FAKE, ldq=64, s=FAKE,
             lds=64, layout=BM, mode=0)
    a.update(kw)
    return lib.mxgg_gather_quant_dim0(a["x"], a["T"], a["cols"], a["ldx"], a["src"], a["K"],
                                      a["rows"], a["q"], a["ldq"], a["s"], a["lds"], a["layout"],
                                      a["mode"], None)


@pytest.mark.parametrize("kw,status", [
    (dict(K=0), _lib.ERR_SHAPE),
    (dict(T=-1), _lib.ERR_SHAPE),
    (dict(cols=48), _lib.ERR_SHAPE),
    (dict(lds=63), _lib.ERR_SHAPE),                    # block-major: lds >= rows
    (dict(ldx=32), _lib.ERR_SHAPE),
    (dict(src=None), _lib.ERR_INVALID_ARGUMENT),
    (dict(x=None), _lib.ERR_INVALID_ARGUMENT),
    (dict(mode=9), _lib.ERR_INVALID_ARGUMENT),
    (dict(layout=7), _lib.ERR_INVALID_ARGUMENT),
    (dict(x=FAKE + 4), _lib.ERR_ALIGNMENT),
    (dict(q=FAKE + 8), _lib.ERR_ALIGNMENT),
    # 65536 column blocks of 512: past the grid's y range
    (dict(cols=65536 * 512, ldx=65536 * 512, ldq=65536 * 512), _lib.ERR_UNSUPPORTED),
])
def test_gather_quant_dim0_rejects(lib, kw, status):
    assert _gather_dim0(lib, **kw) == status


def test_column_counts_above_int32_are_rejected(lib):
    big = 1 << 31   # a multiple of 32; the kernels index columns with 32-bit ints
    assert _gather_dim0(lib, cols=big, ldx=big, ldq=big) == _lib.ERR_UNSUPPORTED
    assert lib.mxgg_quant_dim0(FAKE, 4, big, big, FAKE, big, FAKE, 4, BM, 0, None) == \
        _lib.ERR_UNSUPPORTED
    assert _combine(lib, cols=big, ldy=big, ldo=big) == _lib.ERR_UNSUPPORTED


def test_gather_quant_dim0_empty_is_noop(lib):
    assert _gather_dim0(lib, rows=0) == _lib.OK
    assert _gather_dim0(lib, cols=0) == _lib.OK


def _combine(lib, **kw):
    a = dict(y=FAKE, rows=64, cols=64, ldy=64, perm=FAKE, scores=None, T=16, K=2, out=FAKE, ldo=64)
    a.update(kw)
    return lib.mxgg_combine(a["y"], a["rows"], a["cols"], a["ldy"], a["perm"], a["scores"],
                            a["T"], a["K"], a["out"], a["ldo"], None)


@pytest.mark.parametrize("kw,status", [
    (dict(cols=12), _lib.ERR_SHAPE),
    (dict(K=0), _lib.ERR_SHAPE),
    (dict(ldy=32), _lib.ERR_SHAPE),
    (dict(out=FAKE + 2), _lib.ERR_ALIGNMENT),
    (dict(perm=None), _lib.ERR_INVALID_ARGUMENT),
    (dict(T=1 << 27), _lib.ERR_UNSUPPORTED),
])
def test_combine_rejects(lib, kw, status):
    assert _combine(lib, **kw) == status


def test_combine_empty_is_noop(lib):
    assert _combine(lib, T=0) == _lib.OK


@pytest.mark.parametrize("kw,status", [
    (dict(cols=12), _lib.ERR_SHAPE),
    (dict(K=0), _lib.ERR_SHAPE),
    (dict(y=FAKE + 8), _lib.ERR_ALIGNMENT),
    (dict(perm=None), _lib.ERR_INVALID_ARGUMENT),
    (dict(grad=None), _lib.ERR_INVALID_ARGUMENT),
])
def test_combine_score_grad_rejects(lib, kw, status):
    a = dict(d=FAKE, ldd=64, y=FAKE, rows=64, cols=64, ldy=64, perm=FAKE, T=16, K=2, grad=FAKE)
    a.update(kw)
    assert lib.mxgg_combine_score_grad(a["d"], a["ldd"], a["y"], a["rows"], a["cols"], a["ldy"],
                                       a["perm"], a["T"], a["K"], a["grad"], None) == status


@pytest.mark.parametrize("kw,status", [
    (dict(kind=3), _lib.ERR_INVALID_ARGUMENT),
    (dict(kind=-1), _lib.ERR_INVALID_ARGUMENT),
    (dict(E=0), _lib.ERR_UNSUPPORTED),
    (dict(E=1025), _lib.ERR_UNSUPPORTED),
    (dict(tokens=-1), _lib.ERR_SHAPE),
    (dict(offs=None), _lib.ERR_INVALID_ARGUMENT),
    (dict(ends=None), _lib.ERR_INVALID_ARGUMENT),
    (dict(ends=FAKE), _lib.ERR_INVALID_ARGUMENT),      # aliases offs
])
def test_offs_to_group_ends_rejects(lib, kw, status):
    a = dict(offs=FAKE, E=4, tokens=256, kind=_lib.OFFS_AUTO, ends=FAKE + 64)
    a.update(kw)
    assert lib.mxgg_offs_to_group_ends(a["offs"], a["E"], a["tokens"], a["kind"], a["ends"],
                                       None) == status


@pytest.mark.parametrize("kw,status", [
    (dict(rows=-1), _lib.ERR_SHAPE),
    (dict(ld=16), _lib.ERR_SHAPE),                     # stride below the row
    (dict(E=0), _lib.ERR_UNSUPPORTED),
    (dict(out=None), _lib.ERR_INVALID_ARGUMENT),
    (dict(ends=None), _lib.ERR_INVALID_ARGUMENT),
    (dict(out=FAKE + 8), _lib.ERR_ALIGNMENT),
    (dict(row_bytes=40, ld=48), _lib.ERR_ALIGNMENT),
    (dict(rows=1 << 31), _lib.ERR_UNSUPPORTED),
])
def test_zero_rows_past_groups_rejects(lib, kw, status):
    a = dict(out=FAKE, rows=64, row_bytes=64, ld=64, ends=FAKE, E=2)
    a.update(kw)
    assert lib.mxgg_zero_rows_past_groups(a["out"], a["rows"], a["row_bytes"], a["ld"],
                                          a["ends"], a["E"], None) == status


def test_zero_rows_past_groups_empty_is_noop(lib):
    assert lib.mxgg_zero_rows_past_groups(None, 0, 64, 64, None, 1, None) == _lib.OK
    assert lib.mxgg_zero_rows_past_groups(None, 8, 0, 0, None, 1, None) == _lib.OK
