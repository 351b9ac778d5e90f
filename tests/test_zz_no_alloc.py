"""gtk_layernorm_linear_noalloc through the C ABI against gtk_layernorm_linear
(the workspace form, same kernels): bit-identical outputs on two calls in a
row, the second smaller than the first, for both element types and both
weight layouts; shapes past the static scratch are rejected."""
import ctypes
import os

import numpy as np
import pytest
import torch

from oracle import pair_ops
from tests import helpers as H
from tests.gpu_common import check_bf16, check_fp32, log

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB = os.path.join(ROOT, "genie-tk_amd", "genie_tk", "libgenie_tk_hip.so")
GTK_F32, GTK_BF16 = 0, 1
GTK_W_IN_OUT, GTK_W_OUT_IN = 0, 1
GTK_OK, GTK_EWORKSPACE = 0, 3
SCRATCH_BYTES = 1 << 20

i64, sz, vp, fp, ci = ctypes.c_int64, ctypes.c_size_t, ctypes.c_void_p, ctypes.c_float, ctypes.c_int


@pytest.fixture(scope="module")
def lib():
    L = ctypes.CDLL(LIB)
    L.gtk_last_error.restype = ctypes.c_char_p
    L.gtk_fused_layernorm_linear_workspace_size.restype = sz
    L.gtk_fused_layernorm_linear_workspace_size.argtypes = [i64, i64, ci]
    L.gtk_layernorm_linear.argtypes = [vp, vp, vp, vp, vp, ci, ci, vp, i64, i64, i64, fp, ci,
                                       vp, sz, vp]
    L.gtk_layernorm_linear_noalloc.argtypes = [vp, vp, vp, vp, vp, ci, ci, vp, i64, i64, i64, fp,
                                               ci, vp]
    return L


def _case(lib, rows, d_in, d_out, dtype, layout, with_bias, seed):
    log(f"layernorm_linear_noalloc rows={rows} d_in={d_in} d_out={d_out} {dtype} layout={layout}")
    rng = np.random.default_rng(seed)
    x = (rng.standard_normal((rows, d_in)) * 1.3 + 0.2).astype(np.float32)
    g = (1 + 0.2 * rng.standard_normal(d_in)).astype(np.float32)
    b = (0.2 * rng.standard_normal(d_in)).astype(np.float32)
    w = (rng.standard_normal((d_out, d_in)) / np.sqrt(d_in)).astype(np.float32)  # [out][in]
    bias = rng.standard_normal(d_out).astype(np.float32) if with_bias else None
    tdt, gdt = (torch.bfloat16, GTK_BF16) if dtype == "bf16" else (torch.float32, GTK_F32)
    if dtype == "bf16":
        x, w = H.bf16_round(x), H.bf16_round(w)
    dev = lambda a, t=torch.float32: torch.from_numpy(np.ascontiguousarray(a)).to("cuda", t)  # noqa: E731
    xd, gd, bd = dev(x, tdt), dev(g), dev(b)
    wd = dev(w if layout == GTK_W_OUT_IN else w.T, tdt)
    biasd = dev(bias) if with_bias else None
    y_ws = torch.empty(rows, d_out, device="cuda", dtype=tdt)
    y_na = torch.full((rows, d_out), float("nan"), device="cuda", dtype=tdt)
    ws = torch.empty(lib.gtk_fused_layernorm_linear_workspace_size(d_in, d_out, gdt),
                     device="cuda", dtype=torch.uint8)
    st = torch.cuda.current_stream().cuda_stream
    bptr = biasd.data_ptr() if with_bias else None
    args = (xd.data_ptr(), None, gd.data_ptr(), bd.data_ptr(), wd.data_ptr(), gdt, layout, bptr,
            rows, d_in, d_out, 1e-5, gdt)
    a_ws = list(args)
    a_ws[1] = y_ws.data_ptr()
    a_na = list(args)
    a_na[1] = y_na.data_ptr()
    rc = lib.gtk_layernorm_linear(*a_ws, ws.data_ptr(), ws.numel(), st)
    assert rc == GTK_OK, lib.gtk_last_error()
    rc = lib.gtk_layernorm_linear_noalloc(*a_na, st)
    assert rc == GTK_OK, lib.gtk_last_error()
    torch.cuda.synchronize()
    assert torch.equal(y_na, y_ws), "no-allocation form differs from the workspace form"
    ln = pair_ops.layer_norm(x.astype(np.float64), g, b, 1e-5)
    if dtype == "bf16":
        ln = H.bf16_round(ln.astype(np.float32)).astype(np.float64)
    ref = ln @ w.T.astype(np.float64) + (bias if with_bias else 0.0)
    got = y_na.float().cpu().numpy()
    (check_fp32 if dtype == "fp32" else check_bf16)(got, ref, "layernorm_linear_noalloc")


@pytest.mark.parametrize("dtype", ["bf16", "fp32"])
def test_noalloc_matches_workspace_form(lib, dtype):
    # the first call fills the scratch with a large packed weight; the second,
    # smaller call must not see any of it
    _case(lib, 4133, 256, 1000 if dtype == "bf16" else 900, dtype, GTK_W_OUT_IN, True, 1)
    _case(lib, 77, 64, 40, dtype, GTK_W_IN_OUT, False, 2)
    _case(lib, 300, 128, 128, dtype, GTK_W_OUT_IN, True, 3)


def test_noalloc_rejects_shapes_past_the_scratch(lib):
    need = lib.gtk_fused_layernorm_linear_workspace_size(256, 2017, GTK_BF16)
    assert need > SCRATCH_BYTES
    rc = lib.gtk_layernorm_linear_noalloc(None, None, None, None, None, GTK_BF16, GTK_W_OUT_IN,
                                          None, 10, 256, 2017, 1e-5, GTK_BF16, None)
    assert rc == GTK_EWORKSPACE and b"static array" in lib.gtk_last_error()
    assert lib.gtk_fused_layernorm_linear_workspace_size(256, 2016, GTK_BF16) <= SCRATCH_BYTES
