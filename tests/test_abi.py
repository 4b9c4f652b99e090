"""The C ABI boundary without a GPU: the library loads, exports every function that
include/*.h declares (and the ctypes table binds exactly those), and argument errors are
reported as negative status codes before any HIP call, so no compute runs here.
"""

import ctypes
import re
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
HEADERS = sorted((ROOT / "include").glob("*.h"))


@pytest.fixture(scope="module")
def L(pkg):
    return pkg._lib


@pytest.fixture(scope="module")
def lib(L):
    return L.load()


def header_functions(headers=None) -> set[str]:
    names = set()
    for h in headers or HEADERS:
        text = re.sub(r"/\*.*?\*/", "", h.read_text(), flags=re.S)
        names |= set(re.findall(r"\b(lrq_\w+)\s*\(", text))
    return names


def test_header_parses():
    names = header_functions()
    assert {"lrq_encode", "lrq_decode", "lrq_legacy_encode", "lrq_wht128", "lrq_abi_version"} <= names


def test_test_hooks_stay_out_of_the_dropin_header():
    """The drop-in header declares only entry points with a reference counterpart (or the
    documented additions); test hooks live in lrq_test_hooks.h."""
    main = header_functions([ROOT / "include" / "lrq.h"])
    hooks = header_functions([ROOT / "include" / "lrq_test_hooks.h"])
    assert hooks == {"lrq_encode_twopass"}
    assert not (main & hooks)


def test_every_declared_function_is_exported(L, lib):
    names = header_functions()
    missing = sorted(n for n in names if not hasattr(lib, n))
    assert not missing, missing
    assert not L.missing_symbols()


def test_ctypes_table_matches_header(L):
    assert set(L.SIGNATURES) == header_functions()


def test_abi_version_and_status_strings(lib, L):
    assert lib.lrq_abi_version() == 1
    for code in (L.LRQ_OK, L.LRQ_ERR_NULL, L.LRQ_ERR_SHAPE, L.LRQ_ERR_UNSUPPORTED, L.LRQ_ERR_ALIGN,
                 L.LRQ_ERR_WORKSPACE):
        s = L.status_string(code)
        assert s and s != "unknown status"


def _desc(L, **kw):
    t = L.LrqTensors()
    t.rows, t.hidden, t.rank, t.bits, t.group, t.flags = 32, 4096, 0, 4, 64, 0
    t.codes, t.ld_codes = 4096, 2048
    t.qparams, t.ld_qp = 8192, 128
    for k, v in kw.items():
        setattr(t, k, v)
    return t


def _encode(L, t, x=0x10000, ldx=4096):
    return L.call_raw("lrq_encode", ctypes.byref(t), ctypes.c_void_p(x), ldx, None)


@pytest.mark.parametrize("change,code", [
    (dict(codes=0), "NULL"),
    (dict(bits=3), "UNSUPPORTED"),
    (dict(group=32), "UNSUPPORTED"),
    (dict(rank=8), "UNSUPPORTED"),
    (dict(hidden=4000), "SHAPE"),
    (dict(rows=-1), "SHAPE"),
    (dict(ld_codes=1000), "SHAPE"),
    (dict(ld_codes=2056), "ALIGN"),
    (dict(codes=4097), "ALIGN"),
    (dict(rank=16), "NULL"),                   # rank 16 needs L and V
    (dict(flags=1, group=128), "UNSUPPORTED"),  # rotated int4/g128: rotate with lrq_wht128 first
    (dict(flags=4), "UNSUPPORTED"),
    (dict(n_outlier=3), "NULL"),               # outliers need idx and side
])
def test_encode_argument_errors(L, change, code):
    t = _desc(L, **change)
    assert _encode(L, t) == getattr(L, "LRQ_ERR_" + code)


def test_encode_input_errors(L):
    t = _desc(L)
    assert _encode(L, t, x=0) == L.LRQ_ERR_NULL
    assert _encode(L, t, ldx=100) == L.LRQ_ERR_SHAPE
    assert _encode(L, t, x=0x10002) == L.LRQ_ERR_ALIGN


def test_decode_and_consumer_argument_errors(L):
    t = _desc(L)
    assert L.call_raw("lrq_decode", ctypes.byref(t), None, 4096, None) == L.LRQ_ERR_NULL
    assert L.call_raw("lrq_decode", ctypes.byref(t), ctypes.c_void_p(0x10000), 100, None) == L.LRQ_ERR_SHAPE
    for fn in ("lrq_silu_bwd", "lrq_gelu_bwd", "lrq_mul", "lrq_softmax_bwd"):
        assert L.call_raw(fn, ctypes.byref(t), None, 4096, ctypes.c_void_p(0x10000), 4096, None) == L.LRQ_ERR_NULL
    assert L.call_raw("lrq_dequant_gemm", ctypes.byref(t), ctypes.c_void_p(0x10000), 24,
                      ctypes.c_void_p(0x20000), 24, 1, None) == L.LRQ_ERR_UNSUPPORTED


def test_dequant_gemm_t_arguments(L):
    """Workspace query (host only) and the argument errors of the transposed dequant-GEMM."""
    t = _desc(L)  # 32 rows, 4096 columns, int4 / g64: 32 units -> 32 column groups of 1 unit
    ws = L.call_raw("lrq_dequant_gemm_t_workspace", ctypes.byref(t), 16)
    assert ws == 1 * 4096 * 16 * 4  # 2 row blocks < 8 waves: one row group
    big = _desc(L, rows=16384)
    # 32 column groups -> ceil(256 / 32) = 8 row groups, for n = 16 and n = 32 alike
    assert L.call_raw("lrq_dequant_gemm_t_workspace", ctypes.byref(big), 16) == 8 * 4096 * 16 * 4
    assert L.call_raw("lrq_dequant_gemm_t_workspace", ctypes.byref(big), 32) == 8 * 4096 * 32 * 4
    # rotated: one column group per 128-column rotation block of a plane (16), ceil(256 / 16) = 16 row groups
    assert L.call_raw("lrq_dequant_gemm_t_workspace", ctypes.byref(_desc(L, rows=16384, flags=1)), 32) \
        == 16 * 4096 * 32 * 4
    assert L.call_raw("lrq_dequant_gemm_t_workspace", ctypes.byref(t), 24) == L.LRQ_ERR_UNSUPPORTED
    assert L.call_raw("lrq_dequant_gemm_t_workspace", ctypes.byref(_desc(L, bits=3)), 16) == L.LRQ_ERR_UNSUPPORTED
    p, q = ctypes.c_void_p(0x10000), ctypes.c_void_p(0x20000)
    call = lambda t_, g=p, ldg=16, n=16, o=q, ldo=16, w=ctypes.c_void_p(0x40000), wb=ws: L.call_raw(  # noqa: E731
        "lrq_dequant_gemm_t", ctypes.byref(t_), g, ldg, n, o, ldo, 1, w, wb, None)
    assert call(t, g=None) == L.LRQ_ERR_NULL
    assert call(t, n=24) == L.LRQ_ERR_UNSUPPORTED
    assert call(t, ldg=8) == L.LRQ_ERR_SHAPE
    assert call(t, ldg=18) == L.LRQ_ERR_ALIGN
    assert call(t, g=ctypes.c_void_p(0x10004)) == L.LRQ_ERR_ALIGN
    assert call(t, w=None) == L.LRQ_ERR_NULL
    assert call(t, wb=ws - 4) == L.LRQ_ERR_WORKSPACE
    assert call(t, w=ctypes.c_void_p(0x40008)) == L.LRQ_ERR_ALIGN
    # the rotated format needs planes of whole 128-column rotation blocks (384 / 2 = 192 is not)
    assert call(_desc(L, flags=1, hidden=384)) == L.LRQ_ERR_UNSUPPORTED
    assert L.call_raw("lrq_dequant_gemm_t_workspace", ctypes.byref(_desc(L, flags=1, hidden=384)), 16) \
        == L.LRQ_ERR_UNSUPPORTED


def test_lora_grads_arguments(L):
    """Workspace query (host only) and the argument errors of the one-pass LoRA products."""
    def r16(**kw):
        t_ = _desc(L, rank=16, ld_L=16, V=0x40000, **kw)
        t_.L = 0x30000  # (the descriptor's L field; _desc's own first argument is the library)
        return t_
    big = r16(rows=16384)
    # 32 units -> 8 column groups of 4; 1024 row blocks -> 32 row groups of 32 blocks
    ws = L.call_raw("lrq_lora_grads_workspace", ctypes.byref(big), 16)
    assert ws == 8 * 16384 * 16 * 4 + 32 * 4096 * 16 * 4
    # 32 rows: 2 row groups of one block
    assert L.call_raw("lrq_lora_grads_workspace", ctypes.byref(r16()), 16) == 8 * 32 * 64 + 2 * 4096 * 64
    for t_, n in ((r16(), 32), (_desc(L), 16), (r16(hidden=1792, ld_codes=896, ld_qp=56), 16), (r16(flags=1), 16)):
        assert L.call_raw("lrq_lora_grads_workspace", ctypes.byref(t_), n) == L.LRQ_ERR_UNSUPPORTED
    p = lambda v: ctypes.c_void_p(v)  # noqa: E731
    call = lambda a=p(0x10000), g=p(0x20000), ldg=16, xa=p(0x50000), ldxa=16, da=p(0x60000), w=p(0x70000), wb=ws: (  # noqa: E731
        L.call_raw("lrq_lora_grads", ctypes.byref(big), a, 16, g, ldg, 16, xa, ldxa, 0, da, 16, 1, w, wb, None))
    assert call(a=None) == L.LRQ_ERR_NULL
    assert call(ldg=8) == L.LRQ_ERR_SHAPE
    assert call(g=p(0x20004)) == L.LRQ_ERR_ALIGN
    assert call(ldxa=18) == L.LRQ_ERR_ALIGN
    assert call(da=p(0x60008)) == L.LRQ_ERR_ALIGN  # fp32 da: 16-byte rows
    assert call(w=None) == L.LRQ_ERR_NULL
    assert call(wb=ws - 16) == L.LRQ_ERR_WORKSPACE
    assert call(w=p(0x70008)) == L.LRQ_ERR_ALIGN


def test_coo_and_threshold_arguments(L):
    """Workspace sizes (host only) and argument errors of the outlier compaction, the COO decode
    and the threshold selection."""
    assert L.call_raw("lrq_coo_workspace", 2, 100, 1024) == ((2 * 100 * 16 + 4095) // 4096) * 16
    assert L.call_raw("lrq_coo_workspace", 1, 0, 64) == 0
    assert L.call_raw("lrq_coo_workspace", 1, 4, 0) == L.LRQ_ERR_SHAPE
    p, w = ctypes.c_void_p(0x10000), ctypes.c_void_p(0x40000)
    compact = lambda o=p, cap=64, ld=64, ws=w, wb=16, nnz=p, ptr=p: L.call_raw(  # noqa: E731
        "lrq_coo_compact", o, 1, 16, 512, p, ld, p, cap, nnz, ptr, ws, wb, None)
    assert compact(o=None) == L.LRQ_ERR_NULL
    assert compact(ptr=None) == L.LRQ_ERR_NULL
    assert compact(ld=32) == L.LRQ_ERR_SHAPE             # ld_idx < cap
    assert compact(ws=None) == L.LRQ_ERR_NULL
    assert compact(wb=8) == L.LRQ_ERR_WORKSPACE
    assert compact(nnz=ctypes.c_void_p(0x10004)) == L.LRQ_ERR_ALIGN
    dec = lambda K=16, ptr=p, n=10, cols=p: L.call_raw(  # noqa: E731
        "lrq_legacy_decode_coo", p, p, K, p, ptr, cols, p, n, p, 1, 1, 64, 1024, 4, p, None)
    assert dec(K=8) == L.LRQ_ERR_UNSUPPORTED
    assert dec(ptr=None) == L.LRQ_ERR_NULL
    assert dec(n=-1) == L.LRQ_ERR_SHAPE
    assert dec(cols=None) == L.LRQ_ERR_NULL
    kth = lambda k=5, ws=w, wb=2048, M=64: L.call_raw(  # noqa: E731
        "lrq_legacy_kth_residual", p, p, 16, p, M, 1024, 1024, k, p, ws, wb, None)
    assert kth(k=0) == L.LRQ_ERR_SHAPE
    assert kth(k=64 * 1024 + 1) == L.LRQ_ERR_SHAPE
    assert kth(ws=None) == L.LRQ_ERR_NULL
    assert kth(wb=1024) == L.LRQ_ERR_WORKSPACE
    assert kth(M=1 << 23) == L.LRQ_ERR_SHAPE             # M * N >= 2^32: 32-bit bin counts


def test_legacy_argument_errors(L):
    p = ctypes.c_void_p(0x10000)
    enc = lambda K, bits, N=1024, s_rows=1: L.call_raw(  # noqa: E731
        "lrq_legacy_encode", p, p, K, p, 1, 64, N, 64 * N, N, p, s_rows, bits, 5.0, p, p, None)
    assert enc(8, 4) == L.LRQ_ERR_UNSUPPORTED         # K is padded to 16 / 32 by the caller
    assert enc(16, 3) == L.LRQ_ERR_UNSUPPORTED
    assert enc(16, 4, N=1023) == L.LRQ_ERR_SHAPE      # N % (8 / bits)
    assert enc(16, 4, s_rows=2) == L.LRQ_ERR_SHAPE    # s rows must be 1 or B
    assert L.call_raw("lrq_legacy_decode", None, p, 16, p, None, p, 1, 1, 64, 1024, 4, p, None) == L.LRQ_ERR_NULL
    assert L.call_raw("lrq_legacy_fused", p, p, 16, p, p, 1, 1, 64, 1024, 4, 3, p, p, None) == L.LRQ_ERR_UNSUPPORTED
    assert L.call_raw("lrq_legacy_fused", p, p, 16, p, p, 1, 1, 64, 1024, 4, 1, None, p, None) == L.LRQ_ERR_NULL
    assert L.call_raw("lrq_lowrank_add", p, p, 20, p, 1, 64, 1024, p, None) == L.LRQ_ERR_UNSUPPORTED
    mm = lambda y=p, n=32, ldy=32, ldo=32, K=16, out=p: L.call_raw(  # noqa: E731
        "lrq_legacy_dequant_gemm", p, p, K, p, p, 1, 1, 64, 1024, 2, y, ldy, n, out, ldo, None)
    assert mm(y=None) == L.LRQ_ERR_NULL
    assert mm(out=None) == L.LRQ_ERR_NULL
    assert mm(n=0) == L.LRQ_ERR_SHAPE
    assert mm(ldy=16) == L.LRQ_ERR_SHAPE                 # ldy < n_out
    assert mm(ldo=16) == L.LRQ_ERR_SHAPE
    assert mm(K=8) == L.LRQ_ERR_UNSUPPORTED               # K is padded to 16 / 32 by the caller
    assert mm(y=ctypes.c_void_p(0x10001)) == L.LRQ_ERR_ALIGN


def test_misc_argument_errors(L):
    p = ctypes.c_void_p(0x10000)
    assert L.call_raw("lrq_wht128", p, 1000, 4, 1000, p, 1000, None) == L.LRQ_ERR_SHAPE      # hidden % 128
    assert L.call_raw("lrq_wht128", ctypes.c_void_p(0x10002), 1024, 4, 1024, p, 1024, None) == L.LRQ_ERR_ALIGN
    assert L.call_raw("lrq_wht128", p, 1024, 4, 1024, ctypes.c_void_p(0x10000 + 64), 1024, None) == L.LRQ_ERR_SHAPE
    assert L.call_raw("lrq_dense_elementwise", 7, p, p, p, 100, None) == L.LRQ_ERR_UNSUPPORTED
    assert L.call_raw("lrq_dense_elementwise", 0, None, p, p, 100, None) == L.LRQ_ERR_NULL
    assert L.call_raw("lrq_dense_softmax_bwd", p, p, p, 4, 0, None) == L.LRQ_ERR_SHAPE
    assert L.call_raw("lrq_topk", None, 10, 3, p, None) == L.LRQ_ERR_NULL
    assert L.call_raw("lrq_colmax", p, 10, 4, 100, None, None) == L.LRQ_ERR_NULL


def test_empty_inputs_are_no_ops(L):
    """Zero rows succeed without launching anything (no GPU needed)."""
    t = _desc(L, rows=0)
    assert _encode(L, t) == L.LRQ_OK
    assert L.call_raw("lrq_decode", ctypes.byref(t), ctypes.c_void_p(0x10000), 4096, None) == L.LRQ_OK
    p = ctypes.c_void_p(0x10000)
    assert L.call_raw("lrq_dense_elementwise", 0, p, p, p, 0, None) == L.LRQ_OK
    assert L.call_raw("lrq_wht128", p, 1024, 0, 1024, p, 1024, None) == L.LRQ_OK


def test_header_compiles_as_c_and_a_c_host_links(tmp_path):
    """A plain C host: include/lrq.h compiles as C99 with warnings as errors, links against
    liblrq.so and calls the host-only entry points (no GPU needed)."""
    import shutil
    import subprocess
    cc = shutil.which("gcc")
    if cc is None:
        pytest.skip("no C compiler")
    lib = ROOT / "triton-kernel-test_amd" / "liblrq.so"
    src = tmp_path / "host.c"
    src.write_text(
        '#include <stdio.h>\n#include "lrq.h"\n'
        "int main(void) {\n"
        "  lrq_tensors t = {0};\n"
        "  t.rows = 32; t.hidden = 4096; t.bits = 4; t.group = 64;\n"
        "  t.codes = (void*)0x1000; t.ld_codes = 2048; t.qparams = (void*)0x2000; t.ld_qp = 128;\n"
        "  long long ws = (long long)lrq_dequant_gemm_t_workspace(&t, 16);\n"
        "  long long cw = (long long)lrq_coo_workspace(1, 16, 512);\n"
        '  printf("%d %lld %lld %s\\n", lrq_abi_version(), ws, cw, lrq_status_string(LRQ_ERR_SHAPE));\n'
        "  return lrq_encode(&t, 0, 4096, 0) == LRQ_ERR_NULL ? 0 : 1;\n"
        "}\n")
    exe = tmp_path / "host"
    subprocess.run([cc, "-std=c99", "-Wall", "-Wextra", "-Werror", "-pedantic", f"-I{ROOT / 'include'}", str(src),
                    str(lib), f"-Wl,-rpath,{lib.parent}", "-o", str(exe)], check=True, capture_output=True)
    r = subprocess.run([str(exe)], capture_output=True, text=True, timeout=60)
    assert r.returncode == 0, r.stderr
    ver, ws, cw, msg = r.stdout.split(maxsplit=3)
    assert ver == "1" and int(ws) == 4096 * 16 * 4 and int(cw) == 16 and msg.strip()


def test_host_outlier_indices_are_validated(pkg):
    """Host-held outlier indices (list / numpy / CPU tensor) must be distinct and in [0, hidden)
    (api._outlier_index, before any device work); valid ones come back as int32 unchanged."""
    import torch
    api = pkg.api
    cpu = torch.device("cpu")
    with pytest.raises(ValueError):
        api._outlier_index([3, 4096], 4096, cpu)
    with pytest.raises(ValueError):
        api._outlier_index(torch.tensor([-1, 5]), 4096, cpu)
    with pytest.raises(ValueError):
        api._outlier_index([7, 9, 7], 4096, cpu)
    idx, sanitized = api._outlier_index([9, 0, 4095], 4096, cpu)
    assert not sanitized and idx.dtype == torch.int32 and idx.tolist() == [9, 0, 4095]


def test_row_offset_clamp_stays_in_32_bits():
    """The row clamp of the transposed dequant-GEMM and the LoRA products takes
    min(r * ld, lim * ld) in 32-bit unsigned arithmetic, lim = the block's last present row capped
    at 15.  With strides below 2^24 bytes every term stays below 2^28 for any number of rows,
    so the clamp keeps rows past the end on the last row; without the cap (lim = M - 1 - r0) the
    product wraps once (M - 1 - r0) * ld reaches 2^32 and picks a wrong row."""
    ld = (1 << 24) - 16
    M = 3 * (1 << 16) + 5            # (M - 1 - r0) * ld far above 2^32 at the first blocks
    mask = (1 << 32) - 1
    for r0 in (0, 16 * 1000, 16 * ((M - 1) // 16)):
        for r in range(16):
            want = min(r0 + r, M - 1) - r0   # the clamped row inside the block
            capped = min(M - 1 - r0, 15)
            got = min((r * ld) & mask, (capped * ld) & mask) // ld
            assert got == want
            wrapped = min((r * ld) & mask, ((M - 1 - r0) * ld) & mask) // ld
            if r0 == 0 and r == 15:
                assert wrapped != want       # the uncapped form fails here
