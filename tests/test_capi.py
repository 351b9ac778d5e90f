"""The C ABI (include/genie_tk.h) on the CPU: the shared library loads, exports
every declared entry point, and answers size queries and argument errors
without touching a GPU (validation precedes every HIP call, so no compute is
launched here)."""
import ctypes
import os
import re

import pytest
import torch  # noqa: F401  (the library shares torch's HIP runtime)

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "genie_tk.h")
LIB = os.path.join(ROOT, "genie-tk_amd", "genie_tk", "libgenie_tk_hip.so")

GTK_F32, GTK_BF16 = 0, 1
GTK_OK, GTK_EINVAL, GTK_EUNSUPPORTED, GTK_EWORKSPACE = 0, 1, 2, 3

pytestmark = pytest.mark.skipif(not os.path.exists(LIB), reason="library not built")

i64, sz, vp, fp = ctypes.c_int64, ctypes.c_size_t, ctypes.c_void_p, ctypes.c_float
ci = ctypes.c_int


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(gtk_[a-z0-9_]+)\s*\(", text)))


@pytest.fixture(scope="module")
def lib():
    L = ctypes.CDLL(LIB)
    L.gtk_last_error.restype = ctypes.c_char_p
    for name in ("gtk_triangle_mul_workspace_size", "gtk_tri_mul_workspace_size",
                 "gtk_tri_mul_packed_size", "gtk_tri_attn_packed_size",
                 "gtk_tri_attn_workspace_size", "gtk_triangle_attention_workspace_size",
                 "gtk_fused_layernorm_linear_workspace_size",
                 "gtk_tri_attn_workspace_size_chunked", "gtk_tri_mul_backward_workspace_size",
                 "gtk_tri_mul_workspace_size_chunked", "gtk_pair_transition_packed_size",
                 "gtk_pair_transition_backward_workspace_size",
                 "gtk_tri_attn_backward_workspace_size"):
        getattr(L, name).restype = sz
    L.gtk_triangle_mul_workspace_size.argtypes = [i64, i64, i64, ci]
    L.gtk_tri_mul_workspace_size.argtypes = [i64, i64, i64, i64, ci]
    L.gtk_tri_mul_packed_size.argtypes = [i64, i64, ci]
    L.gtk_tri_attn_packed_size.argtypes = [i64, i64, i64, ci]
    L.gtk_tri_attn_workspace_size.argtypes = [i64, i64, i64, i64, i64, ci]
    L.gtk_tri_mul_backward_workspace_size.argtypes = [i64, i64, i64, i64, ci]
    L.gtk_tri_mul_backward.argtypes = [vp, vp, vp, vp, vp, vp, i64, i64, i64, i64, ci, fp, fp, ci,
                                       vp, sz, vp]
    L.gtk_tri_attn_backward_workspace_size.argtypes = [i64, i64, i64, i64, i64, ci]
    L.gtk_tri_attn_backward.argtypes = [vp, vp, vp, vp, vp, vp, i64, i64, i64, i64, i64, ci, fp,
                                        ci, vp, sz, vp]
    L.gtk_tri_attn_workspace_size_chunked.argtypes = [i64, i64, i64, i64, i64, i64, ci]
    L.gtk_tri_mul_workspace_size_chunked.argtypes = [i64, i64, i64, i64, ci, i64]
    L.gtk_pair_transition_packed_size.argtypes = [i64, i64, ci]
    L.gtk_pair_transition_backward_workspace_size.argtypes = [i64, i64, i64, ci]
    L.gtk_pair_transition_forward.argtypes = [vp, vp, vp, vp, i64, i64, i64, ci, fp, ci, vp]
    L.gtk_pair_transition_backward.argtypes = [vp, vp, vp, vp, vp, i64, i64, i64, fp, ci, vp, sz, vp]
    L.gtk_triangle_attention_workspace_size.argtypes = [i64, i64, i64, i64, ci]
    L.gtk_fused_layernorm_linear_workspace_size.argtypes = [i64, i64, ci]
    L.gtk_layernorm.argtypes = [vp, vp, vp, vp, i64, i64, fp, ci, vp]
    L.gtk_tri_mul_forward.argtypes = [vp, vp, vp, vp, i64, i64, i64, i64, ci, ci, fp, fp, ci,
                                      vp, sz, vp]
    L.gtk_tri_mul_forward_chunked.argtypes = [vp, vp, vp, vp, i64, i64, i64, i64, ci, ci, fp, fp,
                                              ci, i64, vp, sz, vp]
    L.gtk_tri_attn_forward.argtypes = [vp, vp, vp, vp, i64, i64, i64, i64, i64, ci, ci, fp, fp,
                                       ci, vp, sz, vp]
    L.gtk_tri_attn_forward_chunked.argtypes = [vp, vp, vp, vp, i64, i64, i64, i64, i64, ci, ci,
                                               fp, fp, i64, ci, vp, sz, vp]
    L.gtk_triangle_mul_outgoing.argtypes = [vp, vp, vp, vp, i64, i64, i64, ci, vp, sz, vp]
    L.gtk_triangle_attention_starting.argtypes = [vp, vp, vp, vp, vp, fp, vp, i64, i64, i64,
                                                  i64, ci, vp, sz, vp]
    L.gtk_fused_layernorm_linear.argtypes = [vp, vp, vp, vp, vp, ci, vp, i64, i64, i64, fp, ci,
                                             vp, sz, vp]
    L.gtk_layernorm_linear.argtypes = [vp, vp, vp, vp, vp, ci, ci, vp, i64, i64, i64, fp, ci,
                                       vp, sz, vp]
    L.gtk_layernorm_linear_noalloc.argtypes = [vp, vp, vp, vp, vp, ci, ci, vp, i64, i64, i64, fp,
                                               ci, vp]
    L.gtk_timing_report.argtypes = [ctypes.c_char_p, sz]
    return L


def test_header_declares_the_operator_surface():
    names = declared_functions()
    # the reference's _C operators (kernels/bindings.cpp:69-101) and the fused forwards
    for n in ("gtk_layernorm", "gtk_fused_layernorm_linear", "gtk_triangle_mul_outgoing",
              "gtk_triangle_mul_incoming", "gtk_triangle_attention_starting",
              "gtk_triangle_attention_ending", "gtk_tri_mul_forward", "gtk_tri_attn_forward"):
        assert n in names


def test_every_declared_symbol_is_exported(lib):
    missing = [n for n in declared_functions() if not hasattr(lib, n)]
    assert not missing, missing


def test_version_and_error_string(lib):
    assert lib.gtk_version() == 100
    assert isinstance(lib.gtk_last_error(), bytes)


def test_workspace_sizes(lib):
    # three bf16 planes [B][C][Np][Np], Np = N rounded up to 64, 256 B alignment slack
    plane = lambda B, N, C, e: B * C * ((N + 63) // 64 * 64) ** 2 * e
    assert lib.gtk_triangle_mul_workspace_size(1, 512, 128, GTK_BF16) == 3 * (plane(1, 512, 128, 2) + 256)
    assert lib.gtk_triangle_mul_workspace_size(2, 200, 64, GTK_F32) == 3 * (plane(2, 200, 64, 4) + 256)
    # the fused forward pads each channel plane by 256 bytes (power-of-two
    # plane strides put a prologue step's plane stores on the same HBM channels)
    padded = lambda B, N, C, e: B * C * (((N + 63) // 64 * 64) ** 2 * e + 256)
    assert lib.gtk_tri_mul_workspace_size(1, 512, 128, 128, GTK_BF16) == 3 * padded(1, 512, 128, 2) + 3 * 256
    assert lib.gtk_triangle_mul_workspace_size(-1, 8, 16, GTK_F32) == 0
    # tri-mul row chunks: b planes for every row, a and x planes for R rows,
    # R = chunk_rows rounded up to the contraction tile (bf16: 256 rows when
    # Np is a multiple of 256, else 128 or 64; fp32: 128 or 64)
    tc = lambda N, c, dt, rows: lib.gtk_tri_mul_workspace_size_chunked(1, N, 128, c, dt, rows)
    Np = lambda N: (N + 63) // 64 * 64
    chunked = lambda N, c, e, R: c * (Np(N) ** 2 * e + 256) + 2 * c * (R * Np(N) * e + 256) + 3 * 256
    assert tc(2048, 128, GTK_BF16, 0) == tc(2048, 128, GTK_BF16, 2048) == 3 * padded(1, 2048, 128, 2) + 3 * 256
    assert tc(2048, 128, GTK_BF16, 1) == tc(2048, 128, GTK_BF16, 256) == chunked(2048, 128, 2, 256)
    assert tc(2048, 128, GTK_BF16, 300) == chunked(2048, 128, 2, 512)
    assert tc(300, 64, GTK_BF16, 100) == chunked(300, 64, 2, 128)    # Np = 320: 64-row tiles
    assert tc(200, 64, GTK_F32, 100) == chunked(200, 64, 4, 128)     # Np = 256: 128-row tiles (fp32)
    assert tc(2048, 128, GTK_BF16, -1) == 0 and tc(2048, 128, 7, 64) == 0
    # packed weights exist only for the shapes the kernels are built for
    assert lib.gtk_tri_mul_packed_size(128, 128, GTK_BF16) > 0
    assert lib.gtk_tri_mul_packed_size(128, 64, GTK_F32) > lib.gtk_tri_mul_packed_size(128, 64, GTK_BF16)
    assert lib.gtk_tri_mul_packed_size(64, 64, GTK_BF16) > 0
    assert lib.gtk_tri_mul_packed_size(96, 64, GTK_BF16) == 0
    assert lib.gtk_tri_mul_packed_size(64, 48, GTK_BF16) == 0
    assert lib.gtk_tri_attn_packed_size(128, 128, 4, GTK_BF16) > 0
    # heads are padded to 32 channels: d = 8 packs like d = 32
    assert lib.gtk_tri_attn_packed_size(128, 32, 4, GTK_BF16) == lib.gtk_tri_attn_packed_size(128, 128, 4, GTK_BF16)
    assert lib.gtk_tri_attn_packed_size(64, 32, 4, GTK_BF16) > 0
    assert lib.gtk_tri_attn_packed_size(128, 128, 2, GTK_BF16) == 0  # d = 64
    assert lib.gtk_tri_attn_packed_size(128, 64, 8, GTK_BF16) == 0   # 8 heads
    ws = lib.gtk_tri_attn_workspace_size(1, 512, 128, 128, 4, GTK_BF16)
    assert ws >= 4 * 512 * 512 * 128 * 2  # q, k, v^T, gate planes at least
    assert lib.gtk_tri_attn_workspace_size(1, 512, 128, 64, 2, GTK_BF16) > 0
    assert lib.gtk_tri_attn_workspace_size(1, 512, 128, 128, 2, GTK_BF16) == 0
    # row chunks: q, k, v^T and the gate for chunk_rows rows, the triangle
    # bias for all of them; chunk_rows = 0 or >= N is the unchunked size
    wc = lambda rows: lib.gtk_tri_attn_workspace_size_chunked(1, 2048, 128, 128, 4, rows, GTK_BF16)
    full = lib.gtk_tri_attn_workspace_size(1, 2048, 128, 128, 4, GTK_BF16)
    assert wc(0) == full and wc(2048) == full and wc(4096) == full
    assert wc(64) < wc(128) < full
    assert wc(128) - wc(64) == 4 * 64 * 2048 * 128 * 2
    assert full - wc(128) >= 4 * (2048 - 128) * 2048 * 128 * 2
    # every shape and dtype chunks: fp32 and the generic bf16 shapes hold q, k,
    # v and the gate (4 x rows x H*32 x Np) for the chunk's rows only
    wf = lambda rows: lib.gtk_tri_attn_workspace_size_chunked(1, 512, 128, 128, 4, rows, GTK_F32)  # noqa: E731
    assert wf(64) < wf(128) < wf(0) == lib.gtk_tri_attn_workspace_size(1, 512, 128, 128, 4, GTK_F32)
    assert wf(128) - wf(64) == 4 * 64 * 512 * 128 * 4
    wg = lambda rows: lib.gtk_tri_attn_workspace_size_chunked(1, 512, 64, 64, 2, rows, GTK_BF16)  # noqa: E731
    assert wg(64) < wg(0)
    assert lib.gtk_fused_layernorm_linear_workspace_size(128, 256, GTK_BF16) > 0
    # backward: six [c][Np][Np] planes and the per-pair operand planes at least;
    # two more planes where the contraction backward transposes its planes
    # first (fp32, or GENIE_TK_TRANSPOSE_PLANES=1)
    wb = lib.gtk_tri_mul_backward_workspace_size(1, 512, 128, 128, GTK_BF16)
    assert wb >= 6 * plane(1, 512, 128, 2) + 1280 * 512 * 512 * 2
    os.environ["GENIE_TK_TRANSPOSE_PLANES"] = "1"
    try:
        assert lib.gtk_tri_mul_backward_workspace_size(1, 512, 128, 128, GTK_BF16) == wb + 2 * plane(1, 512, 128, 2)
    finally:
        del os.environ["GENIE_TK_TRANSPOSE_PLANES"]
    assert lib.gtk_tri_mul_backward_workspace_size(1, 512, 128, 128, GTK_F32) >= 8 * plane(1, 512, 128, 4)
    assert lib.gtk_tri_mul_backward_workspace_size(1, 512, 128, 96, GTK_BF16) == 0
    # twelve [B][N][H][N][32] activation/gradient buffers at least
    assert lib.gtk_tri_attn_backward_workspace_size(1, 512, 128, 128, 4, GTK_BF16) >= 12 * 512 * 512 * 128 * 2
    assert lib.gtk_tri_attn_backward_workspace_size(1, 512, 128, 64, 4, GTK_BF16) == 0
    # the backward kernels' other shapes: c_z and c in {32, 64, 128}; c_in in {32, 64, 128}
    for cz, c in ((64, 32), (32, 32), (32, 128)):
        assert lib.gtk_tri_mul_backward_workspace_size(1, 64, cz, c, GTK_BF16) > 0
    assert lib.gtk_tri_mul_backward_workspace_size(1, 64, 128, 256, GTK_BF16) == 0
    for cin in (32, 64):
        assert lib.gtk_tri_attn_backward_workspace_size(1, 64, cin, 128, 4, GTK_BF16) > 0
    assert lib.gtk_tri_attn_backward_workspace_size(1, 64, 96, 128, 4, GTK_BF16) == 0


def _err(lib):
    return lib.gtk_last_error().decode()


def test_bad_dtype_and_shapes_are_rejected(lib):
    assert lib.gtk_layernorm(None, None, None, None, 4, 128, 1e-5, 7, None) == GTK_EINVAL
    assert "dtype" in _err(lib)
    assert lib.gtk_layernorm(None, None, None, None, -1, 128, 1e-5, GTK_F32, None) == GTK_EINVAL
    assert lib.gtk_layernorm(None, None, None, None, 4, 128, 1e-5, GTK_F32, None) == GTK_EINVAL
    assert "null" in _err(lib)
    rc = lib.gtk_tri_mul_forward(None, None, None, None, 1, 8, 96, 64, 1, 0, 1e-5, 1e-5,
                                 GTK_BF16, None, 0, None)
    assert rc == GTK_EUNSUPPORTED and "c_z=96" in _err(lib)
    rc = lib.gtk_tri_mul_forward(None, None, None, None, 1, 8, 128, 128, 1, 0, 1e-5, 1e-5,
                                 GTK_BF16, None, 0, None)
    assert rc == GTK_EINVAL and "null" in _err(lib)
    dummy = ctypes.c_void_p(16)  # never dereferenced: the size check fails first
    rc = lib.gtk_tri_mul_forward(dummy, None, dummy, dummy, 1, 8, 128, 128, 1, 0, 1e-5, 1e-5,
                                 GTK_BF16, dummy, 10, None)
    assert rc == GTK_EWORKSPACE and "workspace" in _err(lib)
    rc = lib.gtk_tri_mul_forward_chunked(None, None, None, None, 1, 8, 128, 128, 1, 0, 1e-5, 1e-5,
                                         GTK_BF16, -3, None, 0, None)
    assert rc == GTK_EINVAL and "chunk_rows" in _err(lib)
    # 1.25 GiB (+ alignment, + 256 bytes per channel plane of the b, a and x
    # sets) at 256 rows, 3 GiB unchunked: both checked before any launch
    need = lib.gtk_tri_mul_workspace_size_chunked(1, 2048, 128, 128, GTK_BF16, 256)
    assert need == (5 << 28) + 768 + 3 * 128 * 256
    rc = lib.gtk_tri_mul_forward_chunked(dummy, None, dummy, dummy, 1, 2048, 128, 128, 1, 0, 1e-5,
                                         1e-5, GTK_BF16, 256, dummy, need - 1, None)
    assert rc == GTK_EWORKSPACE and "workspace" in _err(lib)
    rc = lib.gtk_tri_mul_forward(dummy, None, dummy, dummy, 1, 2048, 128, 128, 1, 0, 1e-5, 1e-5,
                                 GTK_BF16, dummy, need, None)
    assert rc == GTK_EWORKSPACE
    rc = lib.gtk_tri_attn_forward(None, None, None, None, 1, 8, 128, 128, 8, 1, 0, 1e-5, 1e9,
                                  GTK_BF16, None, 0, None)
    assert rc == GTK_EUNSUPPORTED
    rc = lib.gtk_tri_attn_forward_chunked(None, None, None, None, 1, 8, 96, 128, 4, 1, 0, 1e-5,
                                          1e9, 4, GTK_F32, None, 0, None)
    assert rc == GTK_EUNSUPPORTED and "c_in=96" in _err(lib)
    rc = lib.gtk_tri_attn_forward_chunked(None, None, None, None, 1, 8, 128, 128, 4, 1, 0, 1e-5,
                                          1e9, -1, GTK_BF16, None, 0, None)
    assert rc == GTK_EINVAL
    for bad in (float("inf"), float("nan"), 2e37):  # the mask bias must stay finite
        rc = lib.gtk_tri_attn_forward(None, None, None, None, 1, 8, 128, 128, 4, 1, 0, 1e-5, bad,
                                      GTK_BF16, None, 0, None)
        assert rc == GTK_EINVAL and "inf" in _err(lib)
    rc = lib.gtk_tri_mul_backward(None, None, None, None, None, None, 1, 8, 128, 96, 1, 1e-5,
                                  1e-5, GTK_BF16, None, 0, None)
    assert rc == GTK_EUNSUPPORTED and "c=96" in _err(lib)
    rc = lib.gtk_tri_mul_backward(None, None, None, None, None, None, 1, 8, 128, 64, 1, 1e-5,
                                  1e-5, GTK_BF16, None, 0, None)
    assert rc == GTK_EINVAL and "null" in _err(lib)
    rc = lib.gtk_tri_attn_backward(None, None, None, None, None, None, 1, 8, 128, 128, 8, 1,
                                   1e-5, GTK_BF16, None, 0, None)
    assert rc == GTK_EUNSUPPORTED and "H=8" in _err(lib)
    rc = lib.gtk_tri_attn_backward(None, None, None, None, None, None, 1, 8, 128, 128, 4, 1,
                                   1e-5, 5, None, 0, None)
    assert rc == GTK_EINVAL and "dtype" in _err(lib)
    rc = lib.gtk_triangle_mul_outgoing(None, None, None, None, 1, 8, 24, GTK_BF16, None, 0, None)
    assert rc == GTK_EUNSUPPORTED and "multiple of 16" in _err(lib)
    rc = lib.gtk_triangle_attention_starting(None, None, None, None, None, 0.2, None, 1, 4, 8,
                                             64, GTK_BF16, None, 0, None)
    assert rc == GTK_EUNSUPPORTED and "head dim" in _err(lib)
    rc = lib.gtk_fused_layernorm_linear(None, None, None, None, None, GTK_F32, None, 4, 96, 8,
                                        1e-5, GTK_F32, None, 0, None)
    assert rc == GTK_EUNSUPPORTED
    rc = lib.gtk_layernorm_linear(None, None, None, None, None, GTK_F32, 2, None, 4, 128, 8,
                                  1e-5, GTK_F32, None, 0, None)
    assert rc == GTK_EINVAL and "layout" in _err(lib)


def test_noalloc_layernorm_linear_validation(lib):
    """The no-allocation form checks its shape against the static scratch
    before any HIP call: too large a packed weight is GTK_EWORKSPACE, an
    empty input succeeds, a null pointer is GTK_EINVAL."""
    rc = lib.gtk_layernorm_linear_noalloc(None, None, None, None, None, GTK_BF16, 1, None, 10,
                                          256, 2017, 1e-5, GTK_BF16, None)
    assert rc == GTK_EWORKSPACE and "static array" in _err(lib)
    rc = lib.gtk_layernorm_linear_noalloc(None, None, None, None, None, GTK_F32, 1, None, 10,
                                          256, 993, 1e-5, GTK_F32, None)
    assert rc == GTK_EWORKSPACE
    assert lib.gtk_layernorm_linear_noalloc(None, None, None, None, None, GTK_BF16, 1, None, 0,
                                            256, 2016, 1e-5, GTK_BF16, None) == GTK_OK
    rc = lib.gtk_layernorm_linear_noalloc(None, None, None, None, None, GTK_BF16, 1, None, 5,
                                          128, 64, 1e-5, GTK_BF16, None)
    assert rc == GTK_EINVAL and "null" in _err(lib)
    rc = lib.gtk_layernorm_linear_noalloc(None, None, None, None, None, GTK_BF16, 1, None, 5,
                                          96, 64, 1e-5, GTK_BF16, None)
    assert rc == GTK_EUNSUPPORTED


def test_empty_inputs_are_no_ops(lib):
    """B = 0 or N = 0 (or rows = 0) succeed without reading any pointer."""
    assert lib.gtk_layernorm(None, None, None, None, 0, 128, 1e-5, GTK_BF16, None) == GTK_OK
    assert lib.gtk_tri_mul_forward(None, None, None, None, 0, 8, 128, 128, 1, 0, 1e-5, 1e-5,
                                   GTK_BF16, None, 0, None) == GTK_OK
    assert lib.gtk_tri_mul_forward(None, None, None, None, 1, 0, 128, 64, 0, 0, 1e-5, 1e-5,
                                   GTK_F32, None, 0, None) == GTK_OK
    assert lib.gtk_tri_attn_forward(None, None, None, None, 2, 0, 128, 128, 4, 0, 0, 1e-5, 1e9,
                                    GTK_BF16, None, 0, None) == GTK_OK
    assert lib.gtk_triangle_mul_outgoing(None, None, None, None, 0, 8, 16, GTK_F32, None, 0,
                                         None) == GTK_OK
    assert lib.gtk_tri_mul_backward(None, None, None, None, None, None, 0, 8, 128, 128, 0, 1e-5,
                                    1e-5, GTK_BF16, None, 0, None) == GTK_OK
    assert lib.gtk_tri_attn_backward(None, None, None, None, None, None, 3, 0, 128, 128, 4, 0,
                                     1e-5, GTK_F32, None, 0, None) == GTK_OK


def test_timing_report_when_idle(lib):
    buf = ctypes.create_string_buffer(256)
    assert lib.gtk_timing_report(buf, 256) == GTK_OK
    assert buf.value == b""


def test_torch_extension_exposes_reference_operators():
    from genie_tk import _ext
    if _ext.C is None:
        pytest.skip(f"extension not built: {_ext.IMPORT_ERROR}")
    for name in ("triangle_mul_outgoing", "triangle_mul_incoming", "triangle_attention_starting",
                 "triangle_attention_ending", "layernorm", "fused_layernorm_linear",
                 "tri_mul_pack", "tri_mul_forward", "tri_attn_pack", "tri_attn_forward"):
        assert hasattr(_ext.C, name), name


class _PtWeights(ctypes.Structure):  # gtk_pair_transition_weights
    _fields_ = [("dtype", ctypes.c_int)] + [(n, ctypes.c_void_p) for n in
                                            ("ln_w", "ln_b", "w1", "b1", "w2", "b2")]


class _PtGrads(ctypes.Structure):  # gtk_pair_transition_grads
    _fields_ = [(n, ctypes.c_void_p) for n in ("ln_w", "ln_b", "w1", "b1", "w2", "b2")]


def test_pair_transition_sizes_and_validation(lib):
    """PairTransition: packed sizes for both dtypes, the backward workspace
    (five channel-major planes at least), and argument checks that fail
    before any launch."""
    bf, f32 = lib.gtk_pair_transition_packed_size(128, 4, GTK_BF16), lib.gtk_pair_transition_packed_size(128, 4, GTK_F32)
    assert 0 < bf < f32
    assert lib.gtk_pair_transition_packed_size(96, 4, GTK_BF16) == 0
    assert lib.gtk_pair_transition_packed_size(128, 2, GTK_F32) == 0
    rows = 4050
    pitch = (rows + 63) // 64 * 64
    ws = lib.gtk_pair_transition_backward_workspace_size(rows, 128, 4, GTK_BF16)
    assert ws >= (3 * 128 + 2 * 512) * pitch * 2
    assert lib.gtk_pair_transition_backward_workspace_size(rows, 128, 4, GTK_F32) > ws
    assert lib.gtk_pair_transition_backward_workspace_size(rows, 96, 4, GTK_BF16) == 0
    assert lib.gtk_pair_transition_backward_workspace_size(-1, 128, 4, GTK_BF16) == 0
    dummy = ctypes.c_void_p(16)  # never dereferenced: every check below fails first
    w = _PtWeights(GTK_F32, *([16] * 6))
    g = _PtGrads(*([None] * 6))
    args = lambda rows, c, dt, wsb: (dummy, dummy, ctypes.byref(w), dummy, ctypes.byref(g), rows, c, 4,  # noqa: E731
                                     1e-5, dt, dummy, wsb, None)
    assert lib.gtk_pair_transition_backward(*args(rows, 128, 7, ws)) == GTK_EINVAL
    assert lib.gtk_pair_transition_backward(*args(rows, 96, GTK_BF16, ws)) == GTK_EUNSUPPORTED
    assert lib.gtk_pair_transition_backward(*args(rows, 128, GTK_BF16, ws - 1)) == GTK_EWORKSPACE
    assert "workspace" in _err(lib)
    assert lib.gtk_pair_transition_backward(*args(0, 128, GTK_BF16, 0)) == GTK_OK
    assert lib.gtk_pair_transition_backward(None, None, ctypes.byref(w), None, ctypes.byref(g), 8, 128, 4,
                                            1e-5, GTK_BF16, None, 0, None) == GTK_EINVAL
    assert lib.gtk_pair_transition_forward(None, None, None, None, 0, 128, 4, 0, 1e-5, GTK_F32, None) == GTK_OK
    assert lib.gtk_pair_transition_forward(None, None, None, None, 8, 128, 4, 0, 1e-5, 5, None) == GTK_EINVAL
