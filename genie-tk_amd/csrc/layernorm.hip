// LayerNorm and LayerNorm+Linear for gfx950.
//
// gtk_layernorm: one pass over HBM.  A row of D channels is spread over D/8
// lanes (8 contiguous channels = 16 B of bf16 per lane), so one wave covers
// 64*8/D rows per step with fully coalesced 16 B loads and stores; U steps
// are issued before any arithmetic so each wave keeps U loads in flight.
// Blocks of 8 waves.  Loads carry the non-temporal hint and stores the
// device-scope policy (written through the L2): measured on MI355X at
// N = 512 / 1024 (bf16, c = 128, inputs in a rotation larger than the MALL,
// launches replayed back to back, variants interleaved), 22.3 / 78.9 us
// against 25.1 / 88.8 us with plain loads and stores, where a plain copy of
// the same bytes took 24.1-24.9 / 87-91 us.  Non-temporal stores, 4- or
// 16-wave blocks and U = 1 or 4 were slower.
// Statistics use an xor-butterfly inside the row's lane group.
//
// gtk_fused_layernorm_linear: the row is normalised in MFMA fragment layout
// (see common.hpp) and multiplied with the packed weight on the matrix cores.
#include <algorithm>
#include <mutex>

#include "capi_util.hpp"
#include "common.hpp"
#include "pack.hpp"

namespace gtk {

template <typename T, int D, int U>
__global__ __launch_bounds__(512) void ln_rows_kernel(const T* __restrict__ x, T* __restrict__ y,
                                                      const float* __restrict__ gamma,
                                                      const float* __restrict__ beta, int64_t rows,
                                                      float eps) {
  constexpr int LPR = D / 8;              // lanes per row
  constexpr int RPW = 64 / LPR;           // rows per wave per step
  constexpr int VEC = 8 * sizeof(T) / 16; // 16-byte pieces per lane and row
  const int lane = threadIdx.x & 63;
  const int wave = wave_id();
  const int sub = lane / LPR;
  const int c0 = (lane % LPR) * 8;
  float g[8], bt[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    g[e] = gamma[c0 + e];
    bt[e] = beta[c0 + e];
  }
  const int64_t wrow0 = ((int64_t)blockIdx.x * 8 + wave) * (RPW * U);  // the wave's first row
  const int64_t row0 = wrow0 + sub;
  // every load is issued before any is used: rows past the last one read
  // the last row (rows >= 1) and are not stored
  uint4 raw_in[U][VEC];
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const int64_t r = row0 + (int64_t)u * RPW;
    const int64_t rc = r < rows ? r : rows - 1;
#pragma unroll
    for (int h = 0; h < VEC; ++h) raw_in[u][h] = load16_nt(x + rc * D + c0 + h * (8 / VEC));
  }
  float v[U][8];
#pragma unroll
  for (int u = 0; u < U; ++u) {
    Frag<T> f;
    __builtin_memcpy(&f, raw_in[u], sizeof(raw_in[u]));
#pragma unroll
    for (int e = 0; e < 8; ++e) v[u][e] = f.get(e);
  }
  // the wave's rows as one buffer range (an empty range for a wave past the
  // last row; rows past the last one take an offset outside the range)
  const int64_t wrows = rows <= wrow0 ? 0 : (rows - wrow0 < RPW * U ? rows - wrow0 : RPW * U);
  const __amdgpu_buffer_rsrc_t out = buf_rsrc(y + wrow0 * D, (uint32_t)(wrows * D * sizeof(T)));
#pragma unroll
  for (int u = 0; u < U; ++u) {
    float s = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) s += v[u][e];
#pragma unroll
    for (int off = LPR / 2; off > 0; off >>= 1) s += __shfl_xor(s, off, 64);
    const float mean = s * (1.0f / D);
    float q = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float d = v[u][e] - mean;
      q += d * d;
    }
#pragma unroll
    for (int off = LPR / 2; off > 0; off >>= 1) q += __shfl_xor(q, off, 64);
    const float rstd = 1.0f / sqrtf(q * (1.0f / D) + eps);
    const int64_t r = row0 + (int64_t)u * RPW;
    float o[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) o[e] = (v[u][e] - mean) * rstd * g[e] + bt[e];
    Frag<T> f;
    f.set(o);
    uint4 raw[VEC];
    __builtin_memcpy(raw, &f, sizeof(raw));
    const uint32_t off = r < rows ? (uint32_t)(((r - wrow0) * D + c0) * sizeof(T)) : kBufSkip;
#pragma unroll
    for (int h = 0; h < VEC; ++h) buf_store16_sc1(out, off + 16u * h, raw[h]);
  }
}

// Any D: one wave per row, three sweeps (sum, centred squares, write).
template <typename T>
__global__ __launch_bounds__(256) void ln_rows_generic_kernel(const T* __restrict__ x,
                                                              T* __restrict__ y,
                                                              const float* __restrict__ gamma,
                                                              const float* __restrict__ beta,
                                                              int64_t rows, int D, float eps) {
  const int lane = threadIdx.x & 63;
  const int64_t r = (int64_t)blockIdx.x * 4 + wave_id();
  if (r >= rows) return;
  const T* xr = x + r * D;
  float s = 0.f;
  for (int c = lane; c < D; c += 64) s += to_f32(xr[c]);
  for (int off = 32; off > 0; off >>= 1) s += __shfl_xor(s, off, 64);
  const float mean = s / (float)D;
  float q = 0.f;
  for (int c = lane; c < D; c += 64) {
    const float d = to_f32(xr[c]) - mean;
    q += d * d;
  }
  for (int off = 32; off > 0; off >>= 1) q += __shfl_xor(q, off, 64);
  const float rstd = 1.0f / sqrtf(q / (float)D + eps);
  for (int c = lane; c < D; c += 64)
    y[r * D + c] = cvt<T>((to_f32(xr[c]) - mean) * rstd * gamma[c] + beta[c]);
}

template <typename T>
static int launch_ln(const T* x, T* y, const float* g, const float* b, int64_t rows, int64_t d,
                     float eps, hipStream_t st) {
  constexpr int U = 2;
  StageTimer timer("layernorm", st);
  auto grid_for = [&](int D) {
    const int64_t rows_per_block = 8 * (64 / (D / 8)) * U;
    return (unsigned)((rows + rows_per_block - 1) / rows_per_block);
  };
  switch (d) {
    case 64: ln_rows_kernel<T, 64, U><<<grid_for(64), 512, 0, st>>>(x, y, g, b, rows, eps); break;
    case 128: ln_rows_kernel<T, 128, U><<<grid_for(128), 512, 0, st>>>(x, y, g, b, rows, eps); break;
    case 256: ln_rows_kernel<T, 256, U><<<grid_for(256), 512, 0, st>>>(x, y, g, b, rows, eps); break;
    case 512: ln_rows_kernel<T, 512, U><<<grid_for(512), 512, 0, st>>>(x, y, g, b, rows, eps); break;
    default:
      ln_rows_generic_kernel<T><<<(unsigned)((rows + 3) / 4), 256, 0, st>>>(x, y, g, b, rows,
                                                                            (int)d, eps);
  }
  GTK_LAUNCH_CHECK();
  return GTK_OK;
}

// ---------------------------------------------------------------------------
// LayerNorm + Linear: y = LN(x) @ W + bias with the LayerNorm affine folded
// in: y = x_hat @ (diag(gamma) W) + (beta @ W + bias), both prepared in the
// workspace (see pack.hpp).  One wave = 32 rows; lane (l&31) owns a row,
// (l>>5) a channel half.
// ---------------------------------------------------------------------------
template <typename T, int DIN>
__global__ __launch_bounds__(256) void ln_linear_kernel(const T* __restrict__ x, T* __restrict__ y,
                                                        const T* __restrict__ wp,
                                                        const float* __restrict__ bias,
                                                        int64_t rows, int d_out, float eps) {
  const int lane = threadIdx.x & 63;
  const int half = lane >> 5;
  const int64_t tile = (int64_t)blockIdx.x * 4 + wave_id();
  const int64_t row = tile * 32 + (lane & 31);
  if (tile * 32 >= rows) return;  // whole wave idle (uniform)
  const bool valid = row < rows;
  RowHalf<DIN> rh;
  load_row_half<T, DIN>(rh, x + (valid ? row : 0) * DIN, valid);
  const f32x2 st = row_stats<DIN>(rh, eps);
  Frag<T> xf[DIN / 16];
  ln_to_frags<T, DIN>(xf, rh, st);
  const int ntiles = (d_out + 31) / 32;
  const bool vec4 = (d_out & 3) == 0;  // 4 outputs per store
  for (int nt = 0; nt < ntiles; ++nt) {
    const f32x16 acc = row_gemm_tile<T, DIN, true>(xf, wp, nt);
    if (!valid) continue;
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const int o0 = nt * 32 + 8 * g + 4 * half;
      if (vec4) {
        if (o0 < d_out)
          store4(y + row * d_out + o0, acc[4 * g] + bias[o0], acc[4 * g + 1] + bias[o0 + 1],
                 acc[4 * g + 2] + bias[o0 + 2], acc[4 * g + 3] + bias[o0 + 3]);
      } else {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int o = o0 + r;
          if (o < d_out) y[row * d_out + o] = cvt<T>(acc[4 * g + r] + bias[o]);
        }
      }
    }
  }
}

// bf16 with the packed weights and the folded bias resident in LDS (dynamic
// shared memory, wbytes + 4 * 32 * ceil(d_out / 32) bytes): persistent blocks
// of 8 waves, one 32-row tile per wave step.  Each output tile's weight
// fragments are read from LDS ahead of its MFMA chain.
template <int DIN>
__global__ __launch_bounds__(512) void ln_linear_lds_kernel(const bf16* __restrict__ x,
                                                            bf16* __restrict__ y,
                                                            const bf16* __restrict__ wp,
                                                            const float* __restrict__ bias,
                                                            int64_t rows, int d_out, float eps,
                                                            int64_t ntiles, int wbytes) {
  extern __shared__ __attribute__((aligned(1024))) char ln_smem[];
  bf16* wl = reinterpret_cast<bf16*>(ln_smem);
  float* bl = reinterpret_cast<float*>(ln_smem + wbytes);
  const int nto = (d_out + 31) / 32;
  copy_to_lds_async(wl, wp, wbytes);
  for (int t = threadIdx.x; t < nto * 32; t += blockDim.x) bl[t] = t < d_out ? bias[t] : 0.f;
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  constexpr int KC = DIN / 16;
  const int lane = threadIdx.x & 63;
  const int half = lane >> 5;
  const int t32 = lane & 31;
  const int wave = wave_id();
  const bool vec4 = (d_out & 3) == 0;
  const int64_t stride = (int64_t)gridDim.x * 8;
  // Rows of a tile; a row past the end (or a tile past the end) reads row 0.
  // The next tile's rows are loaded before this tile's stores, the stores
  // are branch-free (an out-of-range offset drops them) and the first tile
  // is peeled, so the waits for prefetched rows do not wait for stores.
  auto load_rows = [&](Frag<bf16>* raw, int64_t tile) {
    const int64_t row = tile * 32 + t32;
    const bf16* src = x + (row < rows ? row : 0) * DIN + half * (DIN / 2);
#pragma unroll
    for (int ch = 0; ch < KC; ++ch) raw[ch].load(src + ch * 8);
  };
  Frag<bf16> raw[KC];
  auto body = [&](const int64_t tile) {
    const int64_t row = tile * 32 + t32;
    const bool valid = row < rows;
    Frag<bf16> xf[KC];
    ln_frags_bf16<DIN>(xf, raw, eps);
    load_rows(raw, tile + stride);
    const auto ors = buf_rsrc(y + tile * 32 * (int64_t)d_out, (uint32_t)(32 * d_out * 2));
    for (int nt = 0; nt < nto; ++nt) {
      Frag<bf16> f[KC];
#pragma unroll
      for (int ks = 0; ks < KC; ++ks) load_wfrag_lds(f[ks], wl, nt, ks, KC);
      f32x16 acc = mma0(f[0], xf[0]);  // rows = outputs, columns = x rows
#pragma unroll
      for (int ks = 1; ks < KC; ++ks) mma(acc, f[ks], xf[ks]);
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int o0 = nt * 32 + 8 * g + 4 * half;
        const f32x4 b4 = *reinterpret_cast<const f32x4*>(bl + o0);
        if (vec4) {
          const bool ok = valid && o0 < d_out;
          buf_store4(ors, ok ? (uint32_t)((t32 * d_out + o0) * 2) : kBufSkip, acc[4 * g] + b4[0],
                     acc[4 * g + 1] + b4[1], acc[4 * g + 2] + b4[2], acc[4 * g + 3] + b4[3]);
        } else if (valid) {
#pragma unroll
          for (int r = 0; r < 4; ++r)
            if (o0 + r < d_out) y[row * d_out + o0 + r] = (bf16)(acc[4 * g + r] + b4[r]);
        }
      }
    }
  };
  int64_t tile = (int64_t)blockIdx.x * 8 + wave;
  if (tile < ntiles) {
    load_rows(raw, tile);
    body(tile);
    tile += stride;
  }
  for (; tile < ntiles; tile += stride) body(tile);
}

}  // namespace gtk

using namespace gtk;

extern "C" int gtk_layernorm(const void* x, void* y, const float* gamma, const float* beta,
                             int64_t rows, int64_t d, float eps, int dtype, void* stream) {
  GTK_REQUIRE(rows >= 0 && d >= 1, GTK_EINVAL, "gtk_layernorm: bad shape rows=%lld d=%lld",
              (long long)rows, (long long)d);
  GTK_REQUIRE(dtype == GTK_F32 || dtype == GTK_BF16, GTK_EINVAL, "gtk_layernorm: bad dtype %d",
              dtype);
  if (rows == 0) return GTK_OK;
  GTK_REQUIRE(x && y && gamma && beta, GTK_EINVAL, "gtk_layernorm: null pointer");
  GTK_REQUIRE(rows <= (int64_t)1 << 40, GTK_EINVAL, "gtk_layernorm: too many rows");
  hipStream_t st = (hipStream_t)stream;
  if (dtype == GTK_F32) return launch_ln<float>((const float*)x, (float*)y, gamma, beta, rows, d, eps, st);
  return launch_ln<bf16>((const bf16*)x, (bf16*)y, gamma, beta, rows, d, eps, st);
}

// Workspace: packed diag(gamma) W, then the folded bias (fp32, d_out).
template <typename T>
static void carve_ln_linear(Carve& cv, int64_t d_in, int64_t d_out, T** wp, float** bias) {
  *wp = cv.take<T>(packed_elems(d_out, d_in));
  *bias = cv.take<float>(d_out);
}

extern "C" size_t gtk_fused_layernorm_linear_workspace_size(int64_t d_in, int64_t d_out, int dtype) {
  if (d_in < 16 || d_out < 1) return 0;
  Carve cv(nullptr, SIZE_MAX);
  if (dtype == GTK_F32) {
    float* w; float* b;
    carve_ln_linear<float>(cv, d_in, d_out, &w, &b);
  } else {
    bf16* w; float* b;
    carve_ln_linear<bf16>(cv, d_in, d_out, &w, &b);
  }
  return cv.off;
}

extern "C" int gtk_fused_layernorm_linear(const void* x, void* y, const float* gamma,
                                          const float* beta, const void* weight, int weight_dtype,
                                          const float* bias, int64_t rows, int64_t d_in,
                                          int64_t d_out, float eps, int dtype, void* workspace,
                                          size_t workspace_bytes, void* stream) {
  return gtk_layernorm_linear(x, y, gamma, beta, weight, weight_dtype, GTK_W_IN_OUT, bias, rows,
                              d_in, d_out, eps, dtype, workspace, workspace_bytes, stream);
}

extern "C" int gtk_layernorm_linear(const void* x, void* y, const float* gamma, const float* beta,
                                    const void* weight, int weight_dtype, int weight_layout,
                                    const float* bias, int64_t rows, int64_t d_in, int64_t d_out,
                                    float eps, int dtype, void* workspace, size_t workspace_bytes,
                                    void* stream) {
  GTK_REQUIRE(dtype == GTK_F32 || dtype == GTK_BF16, GTK_EINVAL,
              "gtk_fused_layernorm_linear: bad dtype %d", dtype);
  GTK_REQUIRE(weight_layout == GTK_W_IN_OUT || weight_layout == GTK_W_OUT_IN, GTK_EINVAL,
              "gtk_layernorm_linear: bad weight layout %d", weight_layout);
  GTK_REQUIRE(weight_dtype == GTK_F32 || weight_dtype == GTK_BF16, GTK_EINVAL,
              "gtk_fused_layernorm_linear: bad weight dtype %d", weight_dtype);
  GTK_REQUIRE(d_in == 64 || d_in == 128 || d_in == 256, GTK_EUNSUPPORTED,
              "gtk_fused_layernorm_linear: d_in=%lld not in {64,128,256}", (long long)d_in);
  GTK_REQUIRE(d_out >= 1 && d_out <= (1 << 16) && rows >= 0, GTK_EINVAL,
              "gtk_fused_layernorm_linear: bad shape");
  if (rows == 0) return GTK_OK;
  GTK_REQUIRE(x && y && gamma && beta && weight && workspace, GTK_EINVAL,
              "gtk_fused_layernorm_linear: null pointer");
  const size_t need = gtk_fused_layernorm_linear_workspace_size(d_in, d_out, dtype);
  GTK_REQUIRE(workspace_bytes >= need, GTK_EWORKSPACE,
              "gtk_fused_layernorm_linear: workspace %zu < %zu bytes", workspace_bytes, need);
  hipStream_t st = (hipStream_t)stream;
  const unsigned grid = (unsigned)(((rows + 31) / 32 + 3) / 4);
  // Logical W[out][in]: [d_in][d_out] has s_out = 1, s_in = d_out; the
  // nn.Linear layout [d_out][d_in] has s_out = d_in, s_in = 1.
  // The caller's bias has fp32 type; the folded bias starts from it.
  const int64_t s_out = weight_layout == GTK_W_IN_OUT ? 1 : d_in;
  const int64_t s_in = weight_layout == GTK_W_IN_OUT ? d_out : 1;
  int rc;
  Carve cv(workspace, workspace_bytes);
  float* fb;
  if (dtype == GTK_F32) {
    float* wp;
    carve_ln_linear<float>(cv, d_in, d_out, &wp, &fb);
    if ((rc = launch_pack<float>(wp, weight, weight_dtype, (int)d_out, (int)d_in, s_out, s_in, 1.f, st, gamma)))
      return rc;
    if ((rc = launch_fold_bias(fb, weight, nullptr, weight_dtype, beta, (int)d_out, (int)d_in, s_out, s_in, 1.f, st)))
      return rc;
    if (bias && (rc = launch_add_f32(fb, bias, (int)d_out, st))) return rc;
    switch (d_in) {
      case 64: ln_linear_kernel<float, 64><<<grid, 256, 0, st>>>((const float*)x, (float*)y, wp, fb, rows, (int)d_out, eps); break;
      case 128: ln_linear_kernel<float, 128><<<grid, 256, 0, st>>>((const float*)x, (float*)y, wp, fb, rows, (int)d_out, eps); break;
      default: ln_linear_kernel<float, 256><<<grid, 256, 0, st>>>((const float*)x, (float*)y, wp, fb, rows, (int)d_out, eps); break;
    }
  } else {
    bf16* wp;
    carve_ln_linear<bf16>(cv, d_in, d_out, &wp, &fb);
    if ((rc = launch_pack<bf16>(wp, weight, weight_dtype, (int)d_out, (int)d_in, s_out, s_in, 1.f, st, gamma)))
      return rc;
    if ((rc = launch_fold_bias(fb, weight, nullptr, weight_dtype, beta, (int)d_out, (int)d_in, s_out, s_in, 1.f, st)))
      return rc;
    if (bias && (rc = launch_add_f32(fb, bias, (int)d_out, st))) return rc;
    // weights and bias resident in LDS when they fit in 64 KiB
    const int64_t wbytes = packed_elems(d_out, d_in) * 2;
    const int64_t lds = wbytes + ((d_out + 31) / 32) * 32 * 4;
    if (lds <= 64 * 1024) {
      const int64_t ntiles = (rows + 31) / 32;
      StageTimer timer("ln_linear", st);
      const unsigned pgrid = (unsigned)std::min<int64_t>(2 * (int64_t)device_cus(), (ntiles + 7) / 8);
      switch (d_in) {
        case 64: ln_linear_lds_kernel<64><<<pgrid, 512, lds, st>>>((const bf16*)x, (bf16*)y, wp, fb, rows, (int)d_out, eps, ntiles, (int)wbytes); break;
        case 128: ln_linear_lds_kernel<128><<<pgrid, 512, lds, st>>>((const bf16*)x, (bf16*)y, wp, fb, rows, (int)d_out, eps, ntiles, (int)wbytes); break;
        default: ln_linear_lds_kernel<256><<<pgrid, 512, lds, st>>>((const bf16*)x, (bf16*)y, wp, fb, rows, (int)d_out, eps, ntiles, (int)wbytes); break;
      }
      GTK_LAUNCH_CHECK();
      return GTK_OK;
    }
    switch (d_in) {
      case 64: ln_linear_kernel<bf16, 64><<<grid, 256, 0, st>>>((const bf16*)x, (bf16*)y, wp, fb, rows, (int)d_out, eps); break;
      case 128: ln_linear_kernel<bf16, 128><<<grid, 256, 0, st>>>((const bf16*)x, (bf16*)y, wp, fb, rows, (int)d_out, eps); break;
      default: ln_linear_kernel<bf16, 256><<<grid, 256, 0, st>>>((const bf16*)x, (bf16*)y, wp, fb, rows, (int)d_out, eps); break;
    }
  }
  GTK_LAUNCH_CHECK();
  return GTK_OK;
}

// ---------------------------------------------------------------------------
// No-allocation form of gtk_layernorm_linear.  The packed weight and the
// folded bias (its only scratch) go into a file-scope device array instead of
// a caller workspace; each GPU holds its own copy of the array for the life
// of the process.  The array's name is a host-side stand-in in host code: its
// device address is taken once per device with hipGetSymbolAddress and only
// that address is handed to the kernels.  Every call on one GPU shares the
// array, so calls that overlap on one GPU (different streams, or threads)
// race; calls on one stream are ordered.  Each call rewrites every byte the
// kernels read (the packing writes the padding too), so nothing carries over.
// ---------------------------------------------------------------------------
static __device__ __align__(256) char ln_linear_scratch[GTK_LAYERNORM_LINEAR_SCRATCH_BYTES];

namespace {
constexpr int kMaxScratchDevices = 64;
std::mutex g_ln_scratch_mu;
void* g_ln_scratch[kMaxScratchDevices] = {};  // device address of ln_linear_scratch, per device
}  // namespace

static int ln_linear_scratch_ptr(void** out) {
  int dev = -1;
  GTK_HIP_CHECK(hipGetDevice(&dev));
  GTK_REQUIRE(dev >= 0 && dev < kMaxScratchDevices, GTK_EUNSUPPORTED,
              "gtk_layernorm_linear_noalloc: device %d out of range", dev);
  std::lock_guard<std::mutex> lock(g_ln_scratch_mu);
  if (!g_ln_scratch[dev]) {
    void* p = nullptr;
    GTK_HIP_CHECK(hipGetSymbolAddress(&p, HIP_SYMBOL(ln_linear_scratch)));
    GTK_REQUIRE(p != nullptr, GTK_EHIP, "gtk_layernorm_linear_noalloc: no scratch address");
    g_ln_scratch[dev] = p;
  }
  *out = g_ln_scratch[dev];
  return GTK_OK;
}

extern "C" int gtk_layernorm_linear_noalloc(const void* x, void* y, const float* gamma,
                                            const float* beta, const void* weight,
                                            int weight_dtype, int weight_layout, const float* bias,
                                            int64_t rows, int64_t d_in, int64_t d_out, float eps,
                                            int dtype, void* stream) {
  GTK_REQUIRE(dtype == GTK_F32 || dtype == GTK_BF16, GTK_EINVAL,
              "gtk_layernorm_linear_noalloc: bad dtype %d", dtype);
  GTK_REQUIRE(d_in == 64 || d_in == 128 || d_in == 256, GTK_EUNSUPPORTED,
              "gtk_layernorm_linear_noalloc: d_in=%lld not in {64,128,256}", (long long)d_in);
  GTK_REQUIRE(d_out >= 1 && d_out <= (1 << 16) && rows >= 0, GTK_EINVAL,
              "gtk_layernorm_linear_noalloc: bad shape");
  const size_t need = gtk_fused_layernorm_linear_workspace_size(d_in, d_out, dtype);
  GTK_REQUIRE(need <= (size_t)GTK_LAYERNORM_LINEAR_SCRATCH_BYTES, GTK_EWORKSPACE,
              "gtk_layernorm_linear_noalloc: d_in=%lld d_out=%lld needs %zu bytes of scratch, "
              "more than the %zu-byte static array",
              (long long)d_in, (long long)d_out, need, (size_t)GTK_LAYERNORM_LINEAR_SCRATCH_BYTES);
  if (rows == 0) return GTK_OK;
  GTK_REQUIRE(x && y && gamma && beta && weight, GTK_EINVAL,
              "gtk_layernorm_linear_noalloc: null pointer");
  void* scratch = nullptr;
  int rc;
  if ((rc = ln_linear_scratch_ptr(&scratch))) return rc;
  return gtk_layernorm_linear(x, y, gamma, beta, weight, weight_dtype, weight_layout, bias, rows,
                              d_in, d_out, eps, dtype, scratch, GTK_LAYERNORM_LINEAR_SCRATCH_BYTES,
                              stream);
}
