// Weight packing into MFMA fragment order, and small vector conversions.
//
// A weight matrix W (logical [out][in], arbitrary strides) is packed for
// contraction over K = in:
//   dst[((nt*KCH + ks)*64 + l)*8 + e] = scale * W[nt*32 + (l&31)][(l>>5)*K/2 + ks*8 + e]
// with KCH = K/16 chunks and zero rows for out >= OUT.  This is the order the
// device helpers in common.hpp (load_wfrag / row_gemm_tile) read.
#pragma once
#include "capi_util.hpp"
#include "common.hpp"

namespace gtk {

// Grouped padding of one dimension: padded index i is element (i / gp) * g +
// (i % gp) of the source, or zero when i % gp >= g.  Multi-head attention
// pads each head of g channels to gp; {kNoPad, kNoPad} is the identity.
constexpr int kNoPad = 1 << 30;
struct Pad {
  int gp = kNoPad, g = kNoPad;
  __host__ __device__ __forceinline__ int src(int i) const {
    const int q = i / gp, r = i - q * gp;
    return r < g ? q * g + r : -1;
  }
};

inline int64_t packed_elems(int64_t out_dim, int64_t k_dim) {
  return ((out_dim + 31) / 32) * (k_dim / 16) * 512;
}

// `gamma` (optional, fp32 [k_dim]) scales input column k: packing W diag(gamma)
// folds a preceding LayerNorm's elementwise weight into the linear map.
template <typename Tout, typename Tin>
__global__ void pack_weight_kernel(Tout* __restrict__ dst, const Tin* __restrict__ src, int out_dim,
                                   int k_dim, int64_t s_out, int64_t s_in, float scale,
                                   const float* __restrict__ gamma, int64_t total, Pad pout,
                                   Pad pk) {
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= total) return;
  const int kch = k_dim / 16;
  const int e = idx & 7;
  const int l = (idx >> 3) & 63;
  const int64_t rest = idx >> 9;
  const int ks = (int)(rest % kch);
  const int nt = (int)(rest / kch);
  const int o = nt * 32 + (l & 31);
  const int k = (l >> 5) * (k_dim / 2) + ks * 8 + e;
  float v = 0.f;
  const int os = pout.src(o), ksrc = pk.src(k);
  if (o < out_dim && os >= 0 && ksrc >= 0)
    v = scale * to_f32(src[os * s_out + ksrc * s_in]) * (gamma ? gamma[ksrc] : 1.f);
  dst[idx] = cvt<Tout>(v);
}

// dst[o] = scale * (bias[o] + sum_k W[o][k] * beta[k]): the bias of a linear
// map applied after a LayerNorm whose elementwise bias beta is folded in.
// One wave per output: lane l sums k = l, l + 64, ..., then a butterfly over
// the wave (a fixed order, so the result is the same on every call).
constexpr int kFoldWaves = 4;  // outputs per 256-thread block
template <typename Tin>
__global__ __launch_bounds__(64 * kFoldWaves) void fold_bias_kernel(
    float* __restrict__ dst, const Tin* __restrict__ w, const void* __restrict__ bias, int bias_bf16,
    const float* __restrict__ beta, int out_dim, int k_dim, int64_t s_out, int64_t s_in, float scale,
    Pad pout) {
  const int op = blockIdx.x * kFoldWaves + (int)(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (op >= out_dim) return;  // wave-uniform
  const int o = pout.src(op);
  if (o < 0) {
    if (lane == 0) dst[op] = 0.f;
    return;
  }
  float acc = 0.f;
  if (beta)
    for (int k = lane; k < k_dim; k += 64) acc += to_f32(w[o * s_out + k * s_in]) * beta[k];
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) acc += __shfl_xor(acc, off, 64);
  if (lane == 0) {
    const float b = bias ? (bias_bf16 ? (float)((const bf16*)bias)[o] : ((const float*)bias)[o]) : 0.f;
    dst[op] = scale * (b + acc);
  }
}

template <typename Tin>
__global__ void to_f32_kernel(float* __restrict__ dst, const Tin* __restrict__ src, int n,
                              float scale, float fill) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  dst[i] = src ? scale * to_f32(src[i]) : fill;
}

// Pack W (element type `wdtype`) into dst (element type Tout).
template <typename Tout>
inline int launch_pack(Tout* dst, const void* src, int wdtype, int out_dim, int k_dim,
                       int64_t s_out, int64_t s_in, float scale, hipStream_t st,
                       const float* gamma = nullptr, Pad pout = Pad(), Pad pk = Pad()) {
  const int64_t total = packed_elems(out_dim, k_dim);
  const int blocks = (int)((total + 255) / 256);
  if (wdtype == GTK_F32)
    pack_weight_kernel<Tout, float><<<blocks, 256, 0, st>>>(dst, (const float*)src, out_dim, k_dim,
                                                            s_out, s_in, scale, gamma, total, pout, pk);
  else
    pack_weight_kernel<Tout, bf16><<<blocks, 256, 0, st>>>(dst, (const bf16*)src, out_dim, k_dim,
                                                           s_out, s_in, scale, gamma, total, pout, pk);
  GTK_LAUNCH_CHECK();
  return GTK_OK;
}

// Bias of a linear map with a LayerNorm beta folded in (see fold_bias_kernel);
// `bias` has the weights' element type, or is null.
inline int launch_fold_bias(float* dst, const void* w, const void* bias, int wdtype,
                            const float* beta, int out_dim, int k_dim, int64_t s_out, int64_t s_in,
                            float scale, hipStream_t st, Pad pout = Pad()) {
  const int blocks = (out_dim + kFoldWaves - 1) / kFoldWaves;
  if (wdtype == GTK_F32)
    fold_bias_kernel<float><<<blocks, 64 * kFoldWaves, 0, st>>>(dst, (const float*)w, bias, 0, beta,
                                                                 out_dim, k_dim, s_out, s_in, scale, pout);
  else
    fold_bias_kernel<bf16><<<blocks, 64 * kFoldWaves, 0, st>>>(dst, (const bf16*)w, bias, 1, beta,
                                                                out_dim, k_dim, s_out, s_in, scale, pout);
  GTK_LAUNCH_CHECK();
  return GTK_OK;
}

// Convert a parameter vector to fp32 (src == nullptr -> filled with `fill`).
inline int launch_to_f32(float* dst, const void* src, int dtype, int n, float scale, float fill,
                         hipStream_t st) {
  const int blocks = (n + 255) / 256;
  if (dtype == GTK_F32)
    to_f32_kernel<float><<<blocks, 256, 0, st>>>(dst, (const float*)src, n, scale, fill);
  else
    to_f32_kernel<bf16><<<blocks, 256, 0, st>>>(dst, (const bf16*)src, n, scale, fill);
  GTK_LAUNCH_CHECK();
  return GTK_OK;
}

static __global__ void add_f32_kernel(float* __restrict__ dst, const float* __restrict__ src, int n) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) dst[i] += src[i];
}
inline int launch_add_f32(float* dst, const float* src, int n, hipStream_t st) {
  add_f32_kernel<<<(n + 255) / 256, 256, 0, st>>>(dst, src, n);
  GTK_LAUNCH_CHECK();
  return GTK_OK;
}

// Zero a device buffer with a kernel (not hipMemsetAsync, so that callers
// may capture the enqueue into a HIP graph).
static __global__ void zero_fill_kernel(f32x4* __restrict__ p, int64_t n16) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n16) p[i] = f32x4{0.f, 0.f, 0.f, 0.f};
}
inline int launch_zero(void* p, size_t bytes, hipStream_t st) {
  const int64_t n16 = (int64_t)(bytes / 16);
  if (n16 == 0) return GTK_OK;
  zero_fill_kernel<<<(unsigned)((n16 + 255) / 256), 256, 0, st>>>((f32x4*)p, n16);
  GTK_LAUNCH_CHECK();
  return GTK_OK;
}

// Bump allocator over a caller-provided buffer (256-byte aligned slices).
struct Carve {
  char* base;
  size_t cap;
  size_t off = 0;
  Carve(void* b, size_t c) : base((char*)b), cap(c) {}
  template <typename T> T* take(int64_t n) {
    off = (off + 255) & ~size_t(255);
    T* p = (T*)(base ? base + off : nullptr);
    off += sizeof(T) * (size_t)n;
    return p;
  }
  bool fits() const { return off <= cap; }
};

inline size_t dtype_size(int dtype) { return dtype == GTK_F32 ? 4 : 2; }

}  // namespace gtk
