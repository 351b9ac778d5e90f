// Weight packing into MFMA fragment order, and small vector conversions.
//
// A weight matrix W (logical [out][in], arbitrary strides) is packed for
// contraction over K = in:
//   dst[((nt*KCH + ks)*64 + l)*8 + e] = scale * W[nt*32 + (l&31)][(l>>5)*K/2 + ks*8 + e]
// with KCH = K/16 chunks and zero rows for out >= OUT.  This is the order the
// device helpers in common.hpp (load_wfrag / row_gemm_tile) read.
#pragma once
#include <algorithm>

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

// ---------------------------------------------------------------------------
// Batched packing.  A module's packing is a dozen or more tiny launches (each
// a few microseconds of launch latency on the GPU timeline); inside a
// PackScope, launch_to_f32 / launch_pack / launch_pack_acc / launch_fold_bias
// only record their job, and the scope's flush issues one launch per kind,
// in dependency order: the fp32 vectors (LayerNorm parameters that the packs
// and folds read), then every packed matrix, then every folded bias.
// ---------------------------------------------------------------------------
struct WJob {  // one packed matrix
  void* dst;
  const void* src;
  int out_dim, k_dim;
  int64_t s_out, s_in;
  float scale;
  const float* gamma;
  int64_t total;
  Pad pout, pk;
  int acc;  // 1: accumulator k order (launch_pack_acc), 0: fragment order
};
struct FJob {  // one folded bias
  float* dst;
  const void* w;
  const void* bias;
  int bias_bf16;
  const float* beta;
  int out_dim, k_dim;
  int64_t s_out, s_in;
  float scale;
  Pad pout;
};
struct VJob {  // one fp32 vector
  float* dst;
  const void* src;
  int n, src_bf16;
  float scale, fill;
};
constexpr int kPackJobs = 16;
struct WJobs { WJob j[kPackJobs]; };
struct FJobs { FJob j[kPackJobs]; };
struct VJobs { VJob j[kPackJobs]; };

// element idx of a packed matrix: (output row o, input column k) it holds
__device__ __forceinline__ void packed_pos(int64_t idx, int k_dim, int acc, int& o, int& k) {
  const int kch = k_dim / 16;
  const int e = idx & 7;
  const int l = (idx >> 3) & 63;
  const int64_t rest = idx >> 9;
  const int ks = (int)(rest % kch);
  const int nt = (int)(rest / kch);
  o = nt * 32 + (l & 31);
  k = acc ? (ks >> 1) * 32 + 16 * (ks & 1) + 8 * (e >> 2) + 4 * (l >> 5) + (e & 3)
          : (l >> 5) * (k_dim / 2) + ks * 8 + e;
}

template <typename Tout, typename Tin>
__global__ void pack_list_kernel(WJobs L) {
  const WJob J = L.j[blockIdx.y];
  for (int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; idx < J.total;
       idx += (int64_t)gridDim.x * blockDim.x) {
    int o, k;
    packed_pos(idx, J.k_dim, J.acc, o, k);
    float v = 0.f;
    const int os = J.pout.src(o), ksrc = J.pk.src(k);
    if (o < J.out_dim && os >= 0 && ksrc >= 0)
      v = J.scale * to_f32(((const Tin*)J.src)[os * J.s_out + ksrc * J.s_in]) * (J.gamma ? J.gamma[ksrc] : 1.f);
    ((Tout*)J.dst)[idx] = cvt<Tout>(v);
  }
}

template <typename Tin>
__global__ __launch_bounds__(256) void fold_list_kernel(FJobs L) {
  const FJob J = L.j[blockIdx.y];
  const int lane = threadIdx.x & 63;
  for (int op = blockIdx.x * 4 + (int)(threadIdx.x >> 6); op < J.out_dim; op += gridDim.x * 4) {
    const int o = J.pout.src(op);
    if (o < 0) {
      if (lane == 0) J.dst[op] = 0.f;
      continue;
    }
    float acc = 0.f;
    if (J.beta)
      for (int k = lane; k < J.k_dim; k += 64) acc += to_f32(((const Tin*)J.w)[o * J.s_out + k * J.s_in]) * J.beta[k];
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) acc += __shfl_xor(acc, off, 64);
    if (lane == 0) {
      const float b = J.bias ? (J.bias_bf16 ? (float)((const bf16*)J.bias)[o] : ((const float*)J.bias)[o]) : 0.f;
      J.dst[op] = J.scale * (b + acc);
    }
  }
}

static __global__ void vec_list_kernel(VJobs L) {
  const VJob J = L.j[blockIdx.y];
  for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < J.n; i += gridDim.x * blockDim.x)
    J.dst[i] = J.src ? J.scale * (J.src_bf16 ? (float)((const bf16*)J.src)[i] : ((const float*)J.src)[i]) : J.fill;
}

struct PackBatch {
  // matrices by (output type bf16?, input type bf16?)
  WJobs w[2][2];
  int nw[2][2] = {{0, 0}, {0, 0}};
  FJobs f[2];
  int nf[2] = {0, 0};
  VJobs v;
  int nv = 0;
  int64_t wmax[2][2] = {{0, 0}, {0, 0}};
  int fmax[2] = {0, 0}, vmax = 0;
  bool overflow = false;
};
inline PackBatch*& pack_batch() {
  static thread_local PackBatch* b = nullptr;
  return b;
}

inline int flush_pack_batch(PackBatch& b, hipStream_t st) {
  GTK_REQUIRE(!b.overflow, GTK_EINVAL, "packing batch overflow (more than %d jobs of a kind)", kPackJobs);
  if (b.nv) {
    vec_list_kernel<<<dim3((unsigned)((b.vmax + 255) / 256), b.nv), 256, 0, st>>>(b.v);
    GTK_LAUNCH_CHECK();
  }
  auto wl = [&](int to, int ti) -> int {
    if (!b.nw[to][ti]) return GTK_OK;
    const dim3 g((unsigned)std::min<int64_t>((b.wmax[to][ti] + 255) / 256, 1024), b.nw[to][ti]);
    if (to && ti) pack_list_kernel<bf16, bf16><<<g, 256, 0, st>>>(b.w[1][1]);
    else if (to) pack_list_kernel<bf16, float><<<g, 256, 0, st>>>(b.w[1][0]);
    else if (ti) pack_list_kernel<float, bf16><<<g, 256, 0, st>>>(b.w[0][1]);
    else pack_list_kernel<float, float><<<g, 256, 0, st>>>(b.w[0][0]);
    GTK_LAUNCH_CHECK();
    return GTK_OK;
  };
  int rc;
  for (int to = 0; to < 2; ++to)
    for (int ti = 0; ti < 2; ++ti)
      if ((rc = wl(to, ti))) return rc;
  for (int ti = 0; ti < 2; ++ti) {
    if (!b.nf[ti]) continue;
    const dim3 g((unsigned)((b.fmax[ti] + 3) / 4), b.nf[ti]);
    if (ti) fold_list_kernel<bf16><<<g, 256, 0, st>>>(b.f[1]);
    else fold_list_kernel<float><<<g, 256, 0, st>>>(b.f[0]);
    GTK_LAUNCH_CHECK();
  }
  return GTK_OK;
}

// Collects the packing launches of its lifetime (unless an enclosing scope
// already does) and issues them batched at flush().
class PackScope {
 public:
  explicit PackScope(hipStream_t st) : st_(st) {
    if (!pack_batch()) {
      own_ = new PackBatch();
      pack_batch() = own_;
    }
  }
  ~PackScope() {
    if (own_) {
      pack_batch() = nullptr;
      delete own_;
    }
  }
  int flush() {
    if (!own_) return GTK_OK;
    pack_batch() = nullptr;
    const int rc = flush_pack_batch(*own_, st_);
    delete own_;
    own_ = nullptr;
    return rc;
  }

 private:
  hipStream_t st_;
  PackBatch* own_ = nullptr;
};

inline void batch_wjob(PackBatch& b, bool out_bf16, int wdtype, const WJob& j) {
  const int to = out_bf16 ? 1 : 0, ti = wdtype == GTK_F32 ? 0 : 1;
  if (b.nw[to][ti] >= kPackJobs) {
    b.overflow = true;
    return;
  }
  b.w[to][ti].j[b.nw[to][ti]++] = j;
  b.wmax[to][ti] = std::max(b.wmax[to][ti], j.total);
}

// Pack W (element type `wdtype`) into dst (element type Tout).
template <typename Tout>
inline int launch_pack(Tout* dst, const void* src, int wdtype, int out_dim, int k_dim,
                       int64_t s_out, int64_t s_in, float scale, hipStream_t st,
                       const float* gamma = nullptr, Pad pout = Pad(), Pad pk = Pad()) {
  if (PackBatch* b = pack_batch()) {
    batch_wjob(*b, sizeof(Tout) == 2, wdtype,
               WJob{dst, src, out_dim, k_dim, s_out, s_in, scale, gamma, packed_elems(out_dim, k_dim), pout, pk, 0});
    return GTK_OK;
  }
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
  if (PackBatch* b = pack_batch()) {
    const int ti = wdtype == GTK_F32 ? 0 : 1;
    if (b->nf[ti] >= kPackJobs) {
      b->overflow = true;
      return GTK_OK;
    }
    b->f[ti].j[b->nf[ti]++] = FJob{dst, w, bias, ti, beta, out_dim, k_dim, s_out, s_in, scale, pout};
    b->fmax[ti] = std::max(b->fmax[ti], out_dim);
    return GTK_OK;
  }
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
  if (PackBatch* b = pack_batch()) {
    if (b->nv >= kPackJobs) {
      b->overflow = true;
      return GTK_OK;
    }
    b->v.j[b->nv++] = VJob{dst, src, n, dtype == GTK_F32 ? 0 : 1, scale, fill};
    b->vmax = std::max(b->vmax, n);
    return GTK_OK;
  }
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
