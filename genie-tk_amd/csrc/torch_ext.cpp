// genie_tk._C — thin PyTorch binding over the C ABI in include/genie_tk.h.
//
// Mirrors the operator surface of the reference extension
// (kernels/bindings.cpp:69-101: triangle_mul_outgoing/incoming,
// triangle_attention_starting/ending, layernorm, fused_layernorm_linear) and
// adds the fused module entry points used by the modules' _forward_cuda.
// Tensors are checked, made contiguous, and every launch goes to the caller's
// current HIP stream; scratch comes from torch's caching allocator.
#include <c10/hip/HIPStream.h>
#include <torch/extension.h>

#include <vector>

#include "../../include/genie_tk.h"

namespace {

int gtk_dtype_of(const at::Tensor& t, const char* what) {
  if (t.scalar_type() == at::kFloat) return GTK_F32;
  if (t.scalar_type() == at::kBFloat16) return GTK_BF16;
  TORCH_CHECK(false, "genie_tk._C: ", what, " must be float32 or bfloat16, got ", t.scalar_type());
  return -1;
}

void check_rc(int rc) { TORCH_CHECK(rc == GTK_OK, "genie_tk._C: ", gtk_last_error()); }

void* cur_stream(const at::Tensor& t) {
  return (void*)c10::hip::getCurrentHIPStream(t.device().index()).stream();
}

void check_gpu(const at::Tensor& t, const char* what) {
  TORCH_CHECK(t.is_cuda(), what, " must be CUDA tensor");
}

// Every tensor whose data pointer reaches a kernel must live on the device the
// kernels run on (the device of the main input): a host or foreign-device
// pointer would be dereferenced by the GPU.
void check_on(const at::Tensor& t, const at::Tensor& like, const char* what) {
  if (!t.defined()) return;
  TORCH_CHECK(t.device() == like.device(), "genie_tk._C: ", what, " is on ", t.device(),
              " but the input is on ", like.device());
}
void check_on(const c10::optional<at::Tensor>& t, const at::Tensor& like, const char* what) {
  if (t.has_value()) check_on(*t, like, what);
}
void check_all_on(const std::vector<at::Tensor>& ts, const at::Tensor& like, const char* what) {
  for (const auto& t : ts) check_on(t, like, what);
}

at::Tensor f32c(const at::Tensor& t) { return t.to(at::kFloat).contiguous(); }

at::Tensor workspace(const at::Tensor& like, size_t bytes) {
  return at::empty({(int64_t)std::max<size_t>(bytes, 1)}, like.options().dtype(at::kByte));
}

// ---------------------------------------------------------------------------
// Reference operator surface
// ---------------------------------------------------------------------------
at::Tensor layernorm(const at::Tensor& x, const at::Tensor& gamma, const at::Tensor& beta,
                     double eps) {
  check_gpu(x, "x");
  check_on(gamma, x, "gamma");
  check_on(beta, x, "beta");
  const at::DeviceGuard guard(x.device());
  TORCH_CHECK(x.dim() >= 1, "x must have at least one dimension");
  auto xc = x.contiguous();
  const int64_t d = xc.size(-1);
  const int64_t rows = d ? xc.numel() / d : 0;
  auto g = f32c(gamma), b = f32c(beta);
  TORCH_CHECK(g.numel() == d && b.numel() == d, "gamma/beta must have ", d, " elements");
  auto y = at::empty_like(xc);
  check_rc(gtk_layernorm(xc.data_ptr(), y.data_ptr(), g.data_ptr<float>(), b.data_ptr<float>(),
                         rows, d, (float)eps, gtk_dtype_of(xc, "x"), cur_stream(xc)));
  return y;
}

// LayerNorm + Linear over the last dimension of x; weight [D_IN, D_OUT]
// (layout GTK_W_IN_OUT, the reference's operator) or [D_OUT, D_IN]
// (GTK_W_OUT_IN, nn.Linear.weight).
static at::Tensor layernorm_linear_impl(const at::Tensor& x, const at::Tensor& gamma,
                                        const at::Tensor& beta, const at::Tensor& weight,
                                        const c10::optional<at::Tensor>& bias, double eps,
                                        int layout) {
  check_gpu(x, "x");
  check_on(weight, x, "weight");
  check_on(gamma, x, "gamma");
  check_on(beta, x, "beta");
  check_on(bias, x, "bias");
  const at::DeviceGuard guard(x.device());
  auto xc = x.contiguous();
  const int64_t d_in = xc.size(-1);
  const int in_dim = layout == GTK_W_IN_OUT ? 0 : 1;
  TORCH_CHECK(weight.dim() == 2 && weight.size(in_dim) == d_in,
              layout == GTK_W_IN_OUT ? "weight must be [D_IN, D_OUT]" : "weight must be [D_OUT, D_IN]");
  const int64_t d_out = weight.size(1 - in_dim);
  const int64_t rows = d_in ? xc.numel() / d_in : 0;
  auto g = f32c(gamma), b = f32c(beta);
  TORCH_CHECK(g.numel() == d_in && b.numel() == d_in, "gamma/beta must have ", d_in, " elements");
  auto w = weight.contiguous();
  at::Tensor bb;
  if (bias.has_value()) {
    bb = f32c(*bias);
    TORCH_CHECK(bb.numel() == d_out, "bias must have ", d_out, " elements");
  }
  auto sizes = xc.sizes().vec();
  sizes.back() = d_out;
  auto y = at::empty(sizes, xc.options());
  const int dt = gtk_dtype_of(xc, "x");
  auto ws = workspace(xc, gtk_fused_layernorm_linear_workspace_size(d_in, d_out, dt));
  check_rc(gtk_layernorm_linear(xc.data_ptr(), y.data_ptr(), g.data_ptr<float>(),
                                b.data_ptr<float>(), w.data_ptr(), gtk_dtype_of(w, "weight"), layout,
                                bias.has_value() ? bb.data_ptr<float>() : nullptr, rows, d_in, d_out,
                                (float)eps, dt, ws.data_ptr(), ws.numel(), cur_stream(xc)));
  return y;
}

at::Tensor fused_layernorm_linear(const at::Tensor& x, const at::Tensor& gamma,
                                  const at::Tensor& beta, const at::Tensor& weight,
                                  const c10::optional<at::Tensor>& bias, double eps) {
  return layernorm_linear_impl(x, gamma, beta, weight, bias, eps, GTK_W_IN_OUT);
}

at::Tensor layernorm_linear(const at::Tensor& x, const at::Tensor& gamma, const at::Tensor& beta,
                            const at::Tensor& weight, const c10::optional<at::Tensor>& bias,
                            double eps) {
  return layernorm_linear_impl(x, gamma, beta, weight, bias, eps, GTK_W_OUT_IN);
}

at::Tensor triangle_mul_raw(const at::Tensor& a, const at::Tensor& b, const at::Tensor& mask,
                            bool outgoing) {
  check_gpu(a, "a");
  check_on(b, a, "b");
  check_on(mask, a, "mask");
  const at::DeviceGuard guard(a.device());
  TORCH_CHECK(a.dim() == 4 && a.sizes() == b.sizes() && a.size(1) == a.size(2),
              "a and b must both be [B, N, N, C]");
  TORCH_CHECK(a.scalar_type() == b.scalar_type(), "a and b must have the same dtype");
  TORCH_CHECK(mask.numel() == a.size(0) * a.size(1) * a.size(2), "mask must be [B, N, N]");
  auto ac = a.contiguous(), bc = b.contiguous();
  const int64_t B = ac.size(0), N = ac.size(1), C = ac.size(3);
  const int dt = gtk_dtype_of(ac, "a");
  auto x = at::empty_like(ac);
  auto ws = workspace(ac, gtk_triangle_mul_workspace_size(B, N, C, dt));
  auto fn = outgoing ? gtk_triangle_mul_outgoing : gtk_triangle_mul_incoming;
  check_rc(fn(ac.data_ptr(), bc.data_ptr(), nullptr, x.data_ptr(), B, N, C, dt, ws.data_ptr(),
              ws.numel(), cur_stream(ac)));
  return x;
}

at::Tensor triangle_mul_outgoing(const at::Tensor& a, const at::Tensor& b, const at::Tensor& mask) {
  return triangle_mul_raw(a, b, mask, true);
}
at::Tensor triangle_mul_incoming(const at::Tensor& a, const at::Tensor& b, const at::Tensor& mask) {
  return triangle_mul_raw(a, b, mask, false);
}

at::Tensor triangle_attention_raw(const at::Tensor& q, const at::Tensor& k, const at::Tensor& v,
                                  const at::Tensor& bias, const at::Tensor& mask, double scale,
                                  bool starting) {
  check_gpu(q, "q");
  check_on(k, q, "k");
  check_on(v, q, "v");
  check_on(bias, q, "bias");
  check_on(mask, q, "mask");
  const at::DeviceGuard guard(q.device());
  TORCH_CHECK(q.dim() == 5 && q.sizes() == k.sizes() && q.sizes() == v.sizes() &&
                  q.size(2) == q.size(3),
              "q, k, v must be [B, H, N, N, D]");
  TORCH_CHECK(q.scalar_type() == k.scalar_type() && q.scalar_type() == v.scalar_type(),
              "q, k, v must have the same dtype");
  const int64_t B = q.size(0), H = q.size(1), N = q.size(2), D = q.size(4);
  TORCH_CHECK(bias.numel() == B * H * N * N, "bias must be [B, H, N, N]");
  TORCH_CHECK(mask.numel() == B * N * N, "mask must be [B, N, N]");
  auto qc = q.contiguous(), kc = k.contiguous(), vc = v.contiguous();
  auto bc = f32c(bias), mc = f32c(mask);
  const int dt = gtk_dtype_of(qc, "q");
  auto out = at::empty({B, N, N, H * D}, qc.options());
  auto ws = workspace(qc, gtk_triangle_attention_workspace_size(B, H, N, D, dt));
  auto fn = starting ? gtk_triangle_attention_starting : gtk_triangle_attention_ending;
  check_rc(fn(qc.data_ptr(), kc.data_ptr(), vc.data_ptr(), bc.data_ptr<float>(),
              mc.data_ptr<float>(), (float)scale, out.data_ptr(), B, H, N, D, dt, ws.data_ptr(),
              ws.numel(), cur_stream(qc)));
  return out;
}

at::Tensor triangle_attention_starting(const at::Tensor& q, const at::Tensor& k,
                                       const at::Tensor& v, const at::Tensor& bias,
                                       const at::Tensor& mask, double scale) {
  return triangle_attention_raw(q, k, v, bias, mask, scale, true);
}
at::Tensor triangle_attention_ending(const at::Tensor& q, const at::Tensor& k,
                                     const at::Tensor& v, const at::Tensor& bias,
                                     const at::Tensor& mask, double scale) {
  return triangle_attention_raw(q, k, v, bias, mask, scale, false);
}

// ---------------------------------------------------------------------------
// Fused module forwards
// ---------------------------------------------------------------------------
int common_param_dtype(std::vector<at::Tensor>& ps) {
  bool all_bf16 = true;
  for (auto& p : ps)
    if (p.defined() && p.scalar_type() != at::kBFloat16) all_bf16 = false;
  for (auto& p : ps)
    if (p.defined()) p = (all_bf16 ? p : p.to(at::kFloat)).contiguous();
  return all_bf16 ? GTK_BF16 : GTK_F32;
}

const void* ptr_or_null(const at::Tensor& t) { return t.defined() ? t.data_ptr() : nullptr; }

// Parameter gradients as views of one fp32 buffer, each starting 16-byte
// aligned (one allocation; the caller casts them with one conversion of the
// buffer, which follows the views in out).
void flat_grads(std::vector<at::Tensor>& out, const at::Tensor& like,
                const std::vector<std::vector<int64_t>>& shapes, float** const* gs) {
  auto numel = [](const std::vector<int64_t>& s) {
    int64_t n = 1;
    for (auto d : s) n *= d;
    return n;
  };
  int64_t total = 0;
  for (auto& s : shapes) total += (numel(s) + 3) / 4 * 4;
  auto flat = at::empty({total}, like.options().dtype(at::kFloat));
  int64_t o = 0;
  for (size_t i = 0; i < shapes.size(); ++i) {
    const int64_t n = numel(shapes[i]);
    auto t = flat.narrow(0, o, n).view(shapes[i]);
    *gs[i] = t.data_ptr<float>();
    out.push_back(t);
    o += (n + 3) / 4 * 4;
  }
  out.push_back(flat);
}

// params: ln_in_w, ln_in_b, a_p_w, a_p_b, a_g_w, a_g_b, b_p_w, b_p_b, b_g_w, b_g_b,
//         g_w, g_b, ln_out_w, ln_out_b, z_w, z_b
at::Tensor tri_mul_pack(std::vector<at::Tensor> ps, int64_t c_z, int64_t c, bool fp32) {
  TORCH_CHECK(ps.size() == 16, "tri_mul_pack expects 16 parameter tensors");
  check_gpu(ps[2], "weights");
  check_all_on(ps, ps[2], "a parameter");
  const at::DeviceGuard guard(ps[2].device());
  gtk_tri_mul_weights w;
  w.dtype = common_param_dtype(ps);
  const void** slots[16] = {&w.ln_in_w, &w.ln_in_b, &w.a_p_w, &w.a_p_b, &w.a_g_w, &w.a_g_b,
                            &w.b_p_w,   &w.b_p_b,   &w.b_g_w, &w.b_g_b, &w.g_w,   &w.g_b,
                            &w.ln_out_w, &w.ln_out_b, &w.z_w, &w.z_b};
  for (int i = 0; i < 16; ++i) *slots[i] = ptr_or_null(ps[i]);
  const int dt = fp32 ? GTK_F32 : GTK_BF16;
  const size_t bytes = gtk_tri_mul_packed_size(c_z, c, dt);
  TORCH_CHECK(bytes > 0, "genie_tk._C: tri_mul shape c_z=", c_z, " c=", c, " unsupported");
  auto packed = workspace(ps[2], bytes);
  check_rc(gtk_tri_mul_pack(&w, c_z, c, dt, packed.data_ptr(), packed.numel(), cur_stream(ps[2])));
  return packed;
}

// Backward of tri_mul_forward (update only): returns [dz, then the gradients of
// the 16 parameters in tri_mul_pack's order (fp32 views of one buffer), then
// that buffer].
std::vector<at::Tensor> tri_mul_backward(const at::Tensor& z, const c10::optional<at::Tensor>& mask,
                                         const at::Tensor& dy, std::vector<at::Tensor> ps,
                                         int64_t c_z, int64_t c, bool outgoing, double eps_in,
                                         double eps_out) {
  TORCH_CHECK(ps.size() == 16, "tri_mul_backward expects 16 parameter tensors");
  check_gpu(z, "z");
  check_on(mask, z, "mask");
  check_on(dy, z, "dy");
  check_all_on(ps, z, "a parameter");
  const at::DeviceGuard guard(z.device());
  TORCH_CHECK(z.dim() == 4 && z.size(1) == z.size(2) && z.size(3) == c_z, "z must be [B, N, N, c_z]");
  TORCH_CHECK(dy.sizes() == z.sizes() && dy.scalar_type() == z.scalar_type(),
              "dy must match z in shape and dtype");
  auto zc = z.contiguous();
  auto dyc = dy.contiguous();
  const int64_t B = zc.size(0), N = zc.size(1);
  at::Tensor mc;
  if (mask.has_value()) {
    TORCH_CHECK(mask->numel() == B * N * N, "mask must be [B, N, N]");
    mc = f32c(*mask);
  }
  gtk_tri_mul_weights w;
  w.dtype = common_param_dtype(ps);
  const void** slots[16] = {&w.ln_in_w, &w.ln_in_b, &w.a_p_w, &w.a_p_b, &w.a_g_w, &w.a_g_b,
                            &w.b_p_w,   &w.b_p_b,   &w.b_g_w, &w.b_g_b, &w.g_w,   &w.g_b,
                            &w.ln_out_w, &w.ln_out_b, &w.z_w, &w.z_b};
  std::vector<at::Tensor> pc(16);
  for (int i = 0; i < 16; ++i) {
    if (ps[i].defined()) pc[i] = ps[i].contiguous();
    *slots[i] = ptr_or_null(pc[i]);
  }
  const int dt = gtk_dtype_of(zc, "z");
  std::vector<at::Tensor> out;
  out.push_back(at::empty_like(zc));
  gtk_tri_mul_grads g;
  float** gs[16] = {&g.ln_in_w, &g.ln_in_b, &g.a_p_w, &g.a_p_b, &g.a_g_w, &g.a_g_b, &g.b_p_w,
                    &g.b_p_b,   &g.b_g_w,   &g.b_g_b, &g.g_w,   &g.g_b,   &g.ln_out_w,
                    &g.ln_out_b, &g.z_w,    &g.z_b};
  flat_grads(out, zc,
             {{c_z}, {c_z}, {c, c_z}, {c}, {c, c_z}, {c}, {c, c_z}, {c}, {c, c_z}, {c}, {c_z, c_z}, {c_z},
              {c}, {c}, {c_z, c}, {c_z}},
             gs);
  const size_t bytes = gtk_tri_mul_backward_workspace_size(B, N, c_z, c, dt);
  TORCH_CHECK(bytes > 0, "genie_tk._C: tri_mul backward shape c_z=", c_z, " c=", c, " unsupported");
  auto ws = workspace(zc, bytes);
  check_rc(gtk_tri_mul_backward(zc.data_ptr(), mask.has_value() ? mc.data_ptr<float>() : nullptr,
                                dyc.data_ptr(), &w, out[0].data_ptr(), &g, B, N, c_z, c,
                                outgoing ? 1 : 0, (float)eps_in, (float)eps_out, dt, ws.data_ptr(),
                                ws.numel(), cur_stream(zc)));
  return out;
}

// Backward of tri_attn_forward (update only): returns [dx, then the gradients of
// the 10 parameters in tri_attn_pack's order (fp32 views of one buffer), then
// that buffer].
std::vector<at::Tensor> tri_attn_backward(const at::Tensor& x, const c10::optional<at::Tensor>& mask,
                                          const at::Tensor& dy, std::vector<at::Tensor> ps,
                                          int64_t c_in, int64_t c_h, int64_t H, bool starting,
                                          double eps) {
  TORCH_CHECK(ps.size() == 10, "tri_attn_backward expects 10 parameter tensors");
  check_gpu(x, "x");
  check_on(mask, x, "mask");
  check_on(dy, x, "dy");
  check_all_on(ps, x, "a parameter");
  const at::DeviceGuard guard(x.device());
  TORCH_CHECK(x.dim() == 4 && x.size(1) == x.size(2) && x.size(3) == c_in, "x must be [B, N, N, c_in]");
  TORCH_CHECK(dy.sizes() == x.sizes() && dy.scalar_type() == x.scalar_type(),
              "dy must match x in shape and dtype");
  auto xc = x.contiguous();
  auto dyc = dy.contiguous();
  const int64_t B = xc.size(0), N = xc.size(1);
  at::Tensor mc;
  if (mask.has_value()) {
    TORCH_CHECK(mask->numel() == B * N * N, "mask must be [B, N, N]");
    mc = f32c(*mask);
  }
  gtk_tri_attn_weights w;
  w.dtype = common_param_dtype(ps);
  const void** slots[10] = {&w.ln_w, &w.ln_b, &w.tri_w, &w.q_w, &w.k_w,
                            &w.v_w,  &w.g_w,  &w.g_b,   &w.o_w, &w.o_b};
  for (int i = 0; i < 10; ++i) *slots[i] = ptr_or_null(ps[i]);
  const int dt = gtk_dtype_of(xc, "x");
  std::vector<at::Tensor> out;
  out.push_back(at::empty_like(xc));
  gtk_tri_attn_grads g;
  float** gs[10] = {&g.ln_w, &g.ln_b, &g.tri_w, &g.q_w, &g.k_w, &g.v_w, &g.g_w, &g.g_b, &g.o_w, &g.o_b};
  flat_grads(out, xc,
             {{c_in}, {c_in}, {H, c_in}, {c_h, c_in}, {c_h, c_in}, {c_h, c_in}, {c_h, c_in}, {c_h},
              {c_in, c_h}, {c_in}},
             gs);
  const size_t bytes = gtk_tri_attn_backward_workspace_size(B, N, c_in, c_h, H, dt);
  TORCH_CHECK(bytes > 0, "genie_tk._C: tri_attn backward shape c_in=", c_in, " c_h=", c_h, " H=", H,
              " unsupported");
  auto ws = workspace(xc, bytes);
  check_rc(gtk_tri_attn_backward(xc.data_ptr(), mask.has_value() ? mc.data_ptr<float>() : nullptr,
                                 dyc.data_ptr(), &w, out[0].data_ptr(), &g, B, N, c_in, c_h, H,
                                 starting ? 1 : 0, (float)eps, dt, ws.data_ptr(), ws.numel(),
                                 cur_stream(xc)));
  return out;
}

// chunk_rows > 0: the memory-bounded mode (output rows that many at a time)
at::Tensor tri_mul_forward(const at::Tensor& z, const c10::optional<at::Tensor>& mask,
                           const at::Tensor& packed, int64_t c_z, int64_t c, bool outgoing,
                           bool residual, double eps_in, double eps_out, int64_t chunk_rows) {
  check_gpu(z, "z");
  check_on(mask, z, "mask");
  check_on(packed, z, "packed");
  const at::DeviceGuard guard(z.device());
  TORCH_CHECK(z.dim() == 4 && z.size(1) == z.size(2) && z.size(3) == c_z, "z must be [B, N, N, c_z]");
  auto zc = z.contiguous();
  const int64_t B = zc.size(0), N = zc.size(1);
  at::Tensor mc;
  if (mask.has_value()) {
    TORCH_CHECK(mask->numel() == B * N * N, "mask must be [B, N, N]");
    mc = f32c(*mask);
  }
  const int dt = gtk_dtype_of(zc, "z");
  auto out = at::empty_like(zc);
  TORCH_CHECK(chunk_rows >= 0, "tri_mul_forward: chunk_rows must be >= 0");
  auto ws = workspace(zc, gtk_tri_mul_workspace_size_chunked(B, N, c_z, c, dt, chunk_rows));
  check_rc(gtk_tri_mul_forward_chunked(
      zc.data_ptr(), mask.has_value() ? mc.data_ptr<float>() : nullptr, out.data_ptr(),
      packed.data_ptr(), B, N, c_z, c, outgoing ? 1 : 0, residual ? 1 : 0, (float)eps_in,
      (float)eps_out, dt, chunk_rows, ws.data_ptr(), ws.numel(), cur_stream(zc)));
  return out;
}

// The fp8 a/b storage experiment (bf16 z; packed from tri_mul_pack(fp32=False)).
at::Tensor tri_mul_forward_fp8ab(const at::Tensor& z, const c10::optional<at::Tensor>& mask,
                                 const at::Tensor& packed, int64_t c_z, int64_t c, bool outgoing,
                                 bool residual, double eps_in, double eps_out) {
  check_gpu(z, "z");
  check_on(mask, z, "mask");
  check_on(packed, z, "packed");
  const at::DeviceGuard guard(z.device());
  TORCH_CHECK(z.dim() == 4 && z.size(1) == z.size(2) && z.size(3) == c_z, "z must be [B, N, N, c_z]");
  TORCH_CHECK(z.scalar_type() == at::kBFloat16, "tri_mul_forward_fp8ab: bf16 only");
  auto zc = z.contiguous();
  const int64_t B = zc.size(0), N = zc.size(1);
  at::Tensor mc;
  if (mask.has_value()) {
    TORCH_CHECK(mask->numel() == B * N * N, "mask must be [B, N, N]");
    mc = f32c(*mask);
  }
  auto out = at::empty_like(zc);
  const size_t bytes = gtk_tri_mul_fp8ab_workspace_size(B, N, c_z, c);
  TORCH_CHECK(bytes > 0, "tri_mul_forward_fp8ab: shape unsupported");
  auto ws = workspace(zc, bytes);
  check_rc(gtk_tri_mul_forward_fp8ab(zc.data_ptr(), mask.has_value() ? mc.data_ptr<float>() : nullptr,
                                     out.data_ptr(), packed.data_ptr(), B, N, c_z, c, outgoing ? 1 : 0,
                                     residual ? 1 : 0, (float)eps_in, (float)eps_out, ws.data_ptr(),
                                     ws.numel(), cur_stream(zc)));
  return out;
}

// a, b: uint8 [P, Np, Np] (fp8 E4M3 bytes) -> bf16 [P, Np, Np]
at::Tensor tri_mul_contract_fp8(const at::Tensor& a, const at::Tensor& b) {
  check_gpu(a, "a");
  check_on(b, a, "b");
  const at::DeviceGuard guard(a.device());
  TORCH_CHECK(a.scalar_type() == at::kByte && b.scalar_type() == at::kByte, "a, b must be uint8");
  TORCH_CHECK(a.dim() == 3 && a.size(1) == a.size(2) && a.sizes() == b.sizes(), "a, b must be [P, Np, Np]");
  auto ac = a.contiguous(), bc = b.contiguous();
  auto x = at::empty(ac.sizes(), ac.options().dtype(at::kBFloat16));
  check_rc(gtk_tri_mul_contract_fp8(ac.data_ptr(), bc.data_ptr(), x.data_ptr(), ac.size(0), ac.size(1),
                                    cur_stream(ac)));
  return x;
}

// params: ln_w, ln_b, w1, b1, w2, b2 (PairTransition: layer_norm, linear_1, linear_2)
// fp32: pack for the fp32 forward (else bf16)
at::Tensor pair_transition_pack(std::vector<at::Tensor> ps, int64_t c, int64_t n, bool fp32) {
  TORCH_CHECK(ps.size() == 6, "pair_transition_pack expects 6 parameter tensors");
  check_gpu(ps[2], "weights");
  check_all_on(ps, ps[2], "a parameter");
  const at::DeviceGuard guard(ps[2].device());
  gtk_pair_transition_weights w;
  w.dtype = common_param_dtype(ps);
  const void** slots[6] = {&w.ln_w, &w.ln_b, &w.w1, &w.b1, &w.w2, &w.b2};
  for (int i = 0; i < 6; ++i) *slots[i] = ptr_or_null(ps[i]);
  const int dt = fp32 ? GTK_F32 : GTK_BF16;
  const size_t bytes = gtk_pair_transition_packed_size(c, n, dt);
  TORCH_CHECK(bytes > 0, "genie_tk._C: pair_transition shape c=", c, " n=", n, " unsupported");
  auto packed = workspace(ps[2], bytes);
  check_rc(gtk_pair_transition_pack(&w, c, n, dt, packed.data_ptr(), packed.numel(),
                                    cur_stream(ps[2])));
  return packed;
}

// p: [..., c] bf16; mask: [...] (rows of p) or None
at::Tensor pair_transition_forward(const at::Tensor& p, const c10::optional<at::Tensor>& mask,
                                   const at::Tensor& packed, int64_t c, int64_t n, bool residual,
                                   double eps) {
  check_gpu(p, "p");
  check_on(mask, p, "mask");
  check_on(packed, p, "packed");
  const at::DeviceGuard guard(p.device());
  TORCH_CHECK(p.dim() >= 1 && p.size(-1) == c, "p must be [..., c]");
  auto pc = p.contiguous();
  const int dt = gtk_dtype_of(pc, "p");
  const int64_t rows = pc.numel() / c;
  at::Tensor mc;
  if (mask.has_value()) {
    TORCH_CHECK(mask->numel() == rows, "mask must have one value per row of p");
    mc = f32c(*mask);
  }
  auto out = at::empty_like(pc);
  check_rc(gtk_pair_transition_forward(pc.data_ptr(), mask.has_value() ? mc.data_ptr<float>() : nullptr,
                                       out.data_ptr(), packed.data_ptr(), rows, c, n,
                                       residual ? 1 : 0, (float)eps, dt, cur_stream(pc)));
  return out;
}

// Backward of pair_transition_forward (no residual, no mask): returns [dp,
// then the gradients of ln_w, ln_b, w1, b1, w2, b2 (fp32 views of one
// buffer), then that buffer].
std::vector<at::Tensor> pair_transition_backward(const at::Tensor& p, const at::Tensor& dy,
                                                 std::vector<at::Tensor> ps, int64_t c, int64_t n,
                                                 double eps) {
  TORCH_CHECK(ps.size() == 6, "pair_transition_backward expects 6 parameter tensors");
  check_gpu(p, "p");
  check_on(dy, p, "dy");
  check_all_on(ps, p, "a parameter");
  const at::DeviceGuard guard(p.device());
  TORCH_CHECK(p.dim() >= 1 && p.size(-1) == c, "p must be [..., c]");
  TORCH_CHECK(dy.sizes() == p.sizes() && dy.scalar_type() == p.scalar_type(),
              "dy must match p in shape and dtype");
  auto pc = p.contiguous();
  auto dyc = dy.contiguous();
  const int64_t rows = pc.numel() / c;
  gtk_pair_transition_weights w;
  w.dtype = common_param_dtype(ps);
  const void** slots[6] = {&w.ln_w, &w.ln_b, &w.w1, &w.b1, &w.w2, &w.b2};
  std::vector<at::Tensor> prm(6);
  for (int i = 0; i < 6; ++i) {
    if (ps[i].defined()) prm[i] = ps[i].contiguous();
    *slots[i] = ptr_or_null(prm[i]);
  }
  const int dt = gtk_dtype_of(pc, "p");
  std::vector<at::Tensor> out;
  out.push_back(at::empty_like(pc));
  gtk_pair_transition_grads g;
  float** gs[6] = {&g.ln_w, &g.ln_b, &g.w1, &g.b1, &g.w2, &g.b2};
  const int64_t hid = c * n;
  flat_grads(out, pc, {{c}, {c}, {hid, c}, {hid}, {c, hid}, {c}}, gs);
  const size_t bytes = gtk_pair_transition_backward_workspace_size(rows, c, n, dt);
  TORCH_CHECK(bytes > 0, "genie_tk._C: pair_transition backward shape c=", c, " n=", n, " unsupported");
  auto ws = workspace(pc, bytes);
  check_rc(gtk_pair_transition_backward(pc.data_ptr(), dyc.data_ptr(), &w, out[0].data_ptr(), &g,
                                        rows, c, n, (float)eps, dt, ws.data_ptr(), ws.numel(),
                                        cur_stream(pc)));
  return out;
}

// params: ln_w, ln_b, tri_w, q_w, k_w, v_w, g_w, g_b, o_w, o_b
at::Tensor tri_attn_pack(std::vector<at::Tensor> ps, int64_t c_in, int64_t c_h, int64_t H,
                         bool fp32) {
  TORCH_CHECK(ps.size() == 10, "tri_attn_pack expects 10 parameter tensors");
  check_gpu(ps[3], "weights");
  check_all_on(ps, ps[3], "a parameter");
  const at::DeviceGuard guard(ps[3].device());
  gtk_tri_attn_weights w;
  w.dtype = common_param_dtype(ps);
  const void** slots[10] = {&w.ln_w, &w.ln_b, &w.tri_w, &w.q_w, &w.k_w,
                            &w.v_w,  &w.g_w,  &w.g_b,   &w.o_w, &w.o_b};
  for (int i = 0; i < 10; ++i) *slots[i] = ptr_or_null(ps[i]);
  const int dt = fp32 ? GTK_F32 : GTK_BF16;
  const size_t bytes = gtk_tri_attn_packed_size(c_in, c_h, H, dt);
  TORCH_CHECK(bytes > 0, "genie_tk._C: tri_attn shape c_in=", c_in, " c_h=", c_h, " H=", H,
              " unsupported");
  auto packed = workspace(ps[3], bytes);
  check_rc(gtk_tri_attn_pack(&w, c_in, c_h, H, dt, packed.data_ptr(), packed.numel(),
                             cur_stream(ps[3])));
  return packed;
}

at::Tensor tri_attn_forward(const at::Tensor& x, const c10::optional<at::Tensor>& mask,
                            const at::Tensor& packed, int64_t c_in, int64_t c_h, int64_t H,
                            bool starting, bool residual, double eps, int64_t chunk_rows,
                            double inf) {
  check_gpu(x, "x");
  check_on(mask, x, "mask");
  check_on(packed, x, "packed");
  const at::DeviceGuard guard(x.device());
  TORCH_CHECK(x.dim() == 4 && x.size(1) == x.size(2) && x.size(3) == c_in, "x must be [B, N, N, c_in]");
  auto xc = x.contiguous();
  const int64_t B = xc.size(0), N = xc.size(1);
  at::Tensor mc;
  if (mask.has_value()) {
    TORCH_CHECK(mask->numel() == B * N * N, "mask must be [B, N, N]");
    mc = f32c(*mask);
  }
  const int dt = gtk_dtype_of(xc, "x");
  auto out = at::empty_like(xc);
  auto ws = workspace(xc, gtk_tri_attn_workspace_size_chunked(B, N, c_in, c_h, H, chunk_rows, dt));
  check_rc(gtk_tri_attn_forward_chunked(
      xc.data_ptr(), mask.has_value() ? mc.data_ptr<float>() : nullptr, out.data_ptr(),
      packed.data_ptr(), B, N, c_in, c_h, H, starting ? 1 : 0, residual ? 1 : 0, (float)eps,
      (float)inf, chunk_rows, dt, ws.data_ptr(), ws.numel(), cur_stream(xc)));
  return out;
}

py::dict timing_report() {
  std::vector<char> buf(1 << 16);
  check_rc(gtk_timing_report(buf.data(), buf.size()));
  py::dict out;
  const char* p = buf.data();
  while (*p) {
    char name[128];
    int n = 0, used = 0;
    double total = 0, mn = 0, mx = 0;
    if (sscanf(p, "%127s %d %lf %lf %lf%n", name, &n, &total, &mn, &mx, &used) != 5) break;
    out[py::str(name)] = py::make_tuple(n, total, mn, mx);
    p += used;
    while (*p == '\n') ++p;
  }
  return out;
}

}  // namespace

PYBIND11_MODULE(_C, m) {
  m.doc() = "genie_tk._C: gfx950 HIP kernels for the pair-representation hot path";
  m.def("triangle_mul_outgoing", &triangle_mul_outgoing, "Triangle contraction, outgoing edges",
        py::arg("a"), py::arg("b"), py::arg("mask"));
  m.def("triangle_mul_incoming", &triangle_mul_incoming, "Triangle contraction, incoming edges",
        py::arg("a"), py::arg("b"), py::arg("mask"));
  m.def("triangle_attention_starting", &triangle_attention_starting,
        "Triangle attention core, starting node", py::arg("q"), py::arg("k"), py::arg("v"),
        py::arg("bias"), py::arg("mask"), py::arg("scale"));
  m.def("triangle_attention_ending", &triangle_attention_ending,
        "Triangle attention core, ending node", py::arg("q"), py::arg("k"), py::arg("v"),
        py::arg("bias"), py::arg("mask"), py::arg("scale"));
  m.def("layernorm", &layernorm, "LayerNorm forward", py::arg("x"), py::arg("gamma"),
        py::arg("beta"), py::arg("eps") = 1e-5);
  m.def("fused_layernorm_linear", &fused_layernorm_linear, "LayerNorm + Linear forward",
        py::arg("x"), py::arg("gamma"), py::arg("beta"), py::arg("weight"),
        py::arg("bias") = py::none(), py::arg("eps") = 1e-5);
  m.def("layernorm_linear", &layernorm_linear,
        "LayerNorm + Linear forward with an nn.Linear-layout weight [D_OUT, D_IN]", py::arg("x"),
        py::arg("gamma"), py::arg("beta"), py::arg("weight"), py::arg("bias") = py::none(),
        py::arg("eps") = 1e-5);
  m.def("tri_mul_pack", &tri_mul_pack, "Pack TriangleMultiplicativeUpdate parameters",
        py::arg("params"), py::arg("c_z"), py::arg("c"), py::arg("fp32"));
  m.def("tri_mul_forward", &tri_mul_forward, "Fused TriangleMultiplicativeUpdate forward",
        py::arg("z"), py::arg("mask"), py::arg("packed"), py::arg("c_z"), py::arg("c"),
        py::arg("outgoing"), py::arg("residual") = false, py::arg("eps_in") = 1e-5,
        py::arg("eps_out") = 1e-5, py::arg("chunk_rows") = 0);
  m.def("tri_mul_forward_fp8ab", &tri_mul_forward_fp8ab,
        "TriangleMultiplicativeUpdate forward with a and b stored in fp8 E4M3 (experiment)",
        py::arg("z"), py::arg("mask"), py::arg("packed"), py::arg("c_z"), py::arg("c"),
        py::arg("outgoing"), py::arg("residual") = false, py::arg("eps_in") = 1e-5,
        py::arg("eps_out") = 1e-5);
  m.def("tri_mul_contract_fp8", &tri_mul_contract_fp8,
        "x[p] = a[p] . b[p]^T over fp8 E4M3 planes, bf16 out (experiment)", py::arg("a"), py::arg("b"));
  m.def("tri_mul_backward", &tri_mul_backward,
        "TriangleMultiplicativeUpdate backward: [dz, 16 parameter gradients (fp32), their buffer]",
        py::arg("z"), py::arg("mask"), py::arg("dy"), py::arg("params"), py::arg("c_z"),
        py::arg("c"), py::arg("outgoing"), py::arg("eps_in") = 1e-5, py::arg("eps_out") = 1e-5);
  m.def("tri_attn_backward", &tri_attn_backward,
        "TriangleAttention backward: [dx, 10 parameter gradients (fp32), their buffer]", py::arg("x"),
        py::arg("mask"), py::arg("dy"), py::arg("params"), py::arg("c_in"), py::arg("c_h"),
        py::arg("no_heads"), py::arg("starting"), py::arg("eps") = 1e-5);
  m.def("pair_transition_pack", &pair_transition_pack, "Pack PairTransition parameters",
        py::arg("params"), py::arg("c"), py::arg("n"), py::arg("fp32") = false);
  m.def("pair_transition_forward", &pair_transition_forward,
        "Fused PairTransition forward: (residual ? p : 0) + transition(p), times mask",
        py::arg("p"), py::arg("mask"), py::arg("packed"), py::arg("c"), py::arg("n"),
        py::arg("residual") = false, py::arg("eps") = 1e-5);
  m.def("pair_transition_backward", &pair_transition_backward,
        "PairTransition backward: [dp, 6 parameter gradients (fp32), their buffer]", py::arg("p"), py::arg("dy"),
        py::arg("params"), py::arg("c"), py::arg("n"), py::arg("eps") = 1e-5);
  m.def("tri_attn_pack", &tri_attn_pack, "Pack TriangleAttention parameters", py::arg("params"),
        py::arg("c_in"), py::arg("c_h"), py::arg("no_heads"), py::arg("fp32"));
  m.def("tri_attn_forward", &tri_attn_forward, "Fused TriangleAttention forward", py::arg("x"),
        py::arg("mask"), py::arg("packed"), py::arg("c_in"), py::arg("c_h"), py::arg("no_heads"),
        py::arg("starting"), py::arg("residual") = false, py::arg("eps") = 1e-5,
        py::arg("chunk_rows") = 0, py::arg("inf") = 1e9);
  m.def("version", []() { return gtk_version(); });
  m.def("timing_enable", [](bool on) { check_rc(gtk_timing_enable(on ? 1 : 0)); },
        "Record HIP events around every kernel launch (per-kernel timing)", py::arg("on"));
  m.def("timing_report", &timing_report,
        "Wait for recorded kernels; {name: (count, total_ms, min_ms, max_ms)}; clears records");
}
