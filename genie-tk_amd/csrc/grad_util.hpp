// Building blocks shared by the backward passes (tri_mul_bwd.hip,
// tri_attn_bwd.hip).
//
// Per-pair quantities that feed a weight gradient are written channel-major:
// a "CM plane" is [rows][pitch] with element (r, p) = value of channel r at
// pair p, p = (b*N + i)*N + j over the B*N*N pairs, pitch = that count rounded
// up to 64 and the tail columns zero.  Over such planes:
//   * wgrad:   W[m][n] = sum_p G[m][p] X[n][p]   (split over p, fp32 partials)
//   * rowred:  s[r] = sum_p G[r][p],  d[r] = sum_p G[r][p] X[r][p]
//   * fold:    dW[m][n] = W[m][n] gamma[n] + s[m] beta[n], the gradient of a
//     Linear applied to gamma * x_hat + beta when X holds x_hat (the
//     LayerNorm affine is folded into the packed forward weights, so the
//     kernels hold x_hat, not the LayerNorm output).
#pragma once
#include <type_traits>

#include "capi_util.hpp"
#include "common.hpp"
#include "pack.hpp"

namespace gtk {

// Pack W (logical [out][in], strides s_out / s_in) for contraction over K = in
// with the operand taken from MFMA accumulators (SWAP orientation: lane l
// holds pair l&31 and outputs 8g + 4(l>>5) + r of each 32-wide tile).  Chunk
// ks = 2*t + gp, lane half h, element e  <->  k = 32t + 16gp + 8(e>>2) + 4h + (e&3),
// so fragment gp of tile t is acc_t[8gp .. 8gp+7].
template <typename Tout, typename Tin>
__global__ void pack_acc_kernel(Tout* __restrict__ dst, const Tin* __restrict__ src, int out_dim,
                                int k_dim, int64_t s_out, int64_t s_in, int64_t total) {
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= total) return;
  const int kch = k_dim / 16;
  const int e = idx & 7;
  const int l = (idx >> 3) & 63;
  const int64_t rest = idx >> 9;
  const int ks = (int)(rest % kch);
  const int nt = (int)(rest / kch);
  const int k = (ks >> 1) * 32 + 16 * (ks & 1) + 8 * (e >> 2) + 4 * (l >> 5) + (e & 3);
  const int o = nt * 32 + (l & 31);
  dst[idx] = cvt<Tout>(o < out_dim ? to_f32(src[o * s_out + k * s_in]) : 0.f);
}

template <typename Tout>
inline int launch_pack_acc(Tout* dst, const void* src, int wdtype, int out_dim, int k_dim,
                           int64_t s_out, int64_t s_in, hipStream_t st) {
  if (PackBatch* b = pack_batch()) {
    batch_wjob(*b, sizeof(Tout) == 2, wdtype,
               WJob{dst, src, out_dim, k_dim, s_out, s_in, 1.f, nullptr, packed_elems(out_dim, k_dim), Pad(),
                    Pad(), 1});
    return GTK_OK;
  }
  const int64_t total = packed_elems(out_dim, k_dim);
  const int blocks = (int)((total + 255) / 256);
  if (wdtype == GTK_F32)
    pack_acc_kernel<Tout, float><<<blocks, 256, 0, st>>>(dst, (const float*)src, out_dim, k_dim,
                                                         s_out, s_in, total);
  else
    pack_acc_kernel<Tout, bf16><<<blocks, 256, 0, st>>>(dst, (const bf16*)src, out_dim, k_dim,
                                                        s_out, s_in, total);
  GTK_LAUNCH_CHECK();
  return GTK_OK;
}

// Fragments gp = 0, 1 of an accumulator tile, as the A/B operand of the next
// product (pairs as columns, the tile's 32 outputs as k).
template <typename T>
__device__ __forceinline__ void acc_to_frags(Frag<T>* f, const f32x16& acc) {
  float v[16];
#pragma unroll
  for (int e = 0; e < 16; ++e) v[e] = acc[e];
  f[0].set(v);
  f[1].set(v + 8);
}
template <typename T>
__device__ __forceinline__ void vals_to_frags(Frag<T>* f, const float* v) {
  f[0].set(v);
  f[1].set(v + 8);
}

// one bf16 value through a buffer descriptor: byte offset = voff (per lane)
// + soff (wave-uniform, a scalar operand); an offset past the descriptor's
// range reads 0 / drops the store
__device__ __forceinline__ float buf_load_bf16(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
  const unsigned short v = __builtin_amdgcn_raw_buffer_load_b16(r, voff, soff, 0);
  return __uint_as_float((uint32_t)v << 16);
}
__device__ __forceinline__ void buf_store_bf16(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff, float x) {
  __builtin_amdgcn_raw_buffer_store_b16(__builtin_bit_cast(unsigned short, cvt<bf16>(x)), r, voff, soff, 0);
}

// Channel-major rows of a full 32-pair tile through a per-wave LDS tile of
// 32 x 32 bf16 (rows of 72 bytes: the pad spreads both the row writes and the
// transposing reads over the banks).  One 32-channel block then costs two
// 16-byte loads or stores a lane instead of sixteen 2-byte ones.  For tiles
// whose 32 pairs are all valid and whose rows start 16-byte aligned.
constexpr int kCmRow = 36;
constexpr int kCmTile = 32 * kCmRow;
typedef uint32_t cm_u32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t cm_u32x4 __attribute__((ext_vector_type(4)));

// per-lane byte offsets of the 16-byte accesses: cm_store_tile's lane holds
// pairs 8 * (L / 4) .. +7 of channel 4 * G + L % 4 (L = lane % 16,
// G = lane / 16); cm_load_tile's lane reads pairs 8 * (lane % 4) .. +7 of
// channel lane / 4 (and 16 + lane / 4)
__device__ __forceinline__ uint32_t cm_store_voff(int64_t stride) {
  const int lane = threadIdx.x & 63, L = lane & 15, G = lane >> 4;
  return (uint32_t)((4 * G + (L & 3)) * stride + 8 * (L >> 2)) * 2;
}
__device__ __forceinline__ uint32_t cm_load_voff(int64_t stride) {
  const int lane = threadIdx.x & 63;
  return (uint32_t)((lane >> 2) * stride + 8 * (lane & 3)) * 2;
}

// accumulator values of a 32-channel block (value 4g + r: channel
// 8g + 4 * half + r of pair lane % 32) -> the block's 32 rows at byte offset
// soff (channel 0 of the block) + voff; rows are stride elements apart
__device__ __forceinline__ void cm_store_tile(bf16* sw, const float* v, __amdgpu_buffer_rsrc_t r, uint32_t voff,
                                              uint32_t soff, int64_t stride) {
  const int lane = threadIdx.x & 63, half = lane >> 5, t32 = lane & 31;
  const int L = lane & 15, G = lane >> 4;
  __builtin_amdgcn_wave_barrier();
#pragma unroll
  for (int g = 0; g < 4; ++g)
    *reinterpret_cast<cm_u32x2*>(sw + t32 * kCmRow + 8 * g + 4 * half) =
        cm_u32x2{pack_bf16x2(v[4 * g], v[4 * g + 1]), pack_bf16x2(v[4 * g + 2], v[4 * g + 3])};
  __builtin_amdgcn_wave_barrier();
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    // supplier L: pair row 8 * (L % 4) + 4e + L / 4, channels 16h + 4G .. +3
    const s16x4 p0 = lds_read_tr16(sw + (8 * (L & 3) + (L >> 2)) * kCmRow + 16 * h + 4 * G);
    const s16x4 p1 = lds_read_tr16(sw + (8 * (L & 3) + 4 + (L >> 2)) * kCmRow + 16 * h + 4 * G);
    const cm_u32x4 q = __builtin_bit_cast(cm_u32x4, __builtin_shufflevector(p0, p1, 0, 1, 2, 3, 4, 5, 6, 7));
    __builtin_amdgcn_raw_buffer_store_b128(q, r, voff, soff + (uint32_t)(16 * h * stride) * 2, 0);
  }
}

// the 32 rows of a block at byte offset soff + voff -> accumulator values
__device__ __forceinline__ void cm_load_tile(bf16* sw, float* v, __amdgpu_buffer_rsrc_t r, uint32_t voff,
                                             uint32_t soff, int64_t stride) {
  const int lane = threadIdx.x & 63, half = lane >> 5;
  const int L = lane & 15, G = lane >> 4;
  const cm_u32x4 a = __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, 0);
  const cm_u32x4 b = __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff + (uint32_t)(16 * stride) * 2, 0);
  __builtin_amdgcn_wave_barrier();
  bf16* const w0 = sw + (lane >> 2) * kCmRow + 8 * (lane & 3);
  *reinterpret_cast<cm_u32x2*>(w0) = cm_u32x2{a[0], a[1]};
  *reinterpret_cast<cm_u32x2*>(w0 + 4) = cm_u32x2{a[2], a[3]};
  *reinterpret_cast<cm_u32x2*>(w0 + 16 * kCmRow) = cm_u32x2{b[0], b[1]};
  *reinterpret_cast<cm_u32x2*>(w0 + 16 * kCmRow + 4) = cm_u32x2{b[2], b[3]};
  __builtin_amdgcn_wave_barrier();
#pragma unroll
  for (int g = 0; g < 4; ++g) {
    // supplier L: channel row 8g + 4 * half + L / 4, pairs 16 * (G % 2) + 4 * (L % 4) .. +3
    const s16x4 p = lds_read_tr16(sw + (8 * g + 4 * half + (L >> 2)) * kCmRow + 16 * (G & 1) + 4 * (L & 3));
#pragma unroll
    for (int k = 0; k < 4; ++k) v[4 * g + k] = __uint_as_float((uint32_t)(unsigned short)p[k] << 16);
  }
}


// The same with plain pointers: base = channel 0 of the block at the tile's
// first position (16-byte aligned), rows stride elements apart.
__device__ __forceinline__ void cm_store_tile(bf16* sw, const float* v, bf16* base, int64_t stride) {
  const int lane = threadIdx.x & 63, half = lane >> 5, t32 = lane & 31;
  const int L = lane & 15, G = lane >> 4;
  __builtin_amdgcn_wave_barrier();
#pragma unroll
  for (int g = 0; g < 4; ++g)
    *reinterpret_cast<cm_u32x2*>(sw + t32 * kCmRow + 8 * g + 4 * half) =
        cm_u32x2{pack_bf16x2(v[4 * g], v[4 * g + 1]), pack_bf16x2(v[4 * g + 2], v[4 * g + 3])};
  __builtin_amdgcn_wave_barrier();
  bf16* const dst = base + (4 * G + (L & 3)) * stride + 8 * (L >> 2);
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const s16x4 p0 = lds_read_tr16(sw + (8 * (L & 3) + (L >> 2)) * kCmRow + 16 * h + 4 * G);
    const s16x4 p1 = lds_read_tr16(sw + (8 * (L & 3) + 4 + (L >> 2)) * kCmRow + 16 * h + 4 * G);
    *reinterpret_cast<cm_u32x4*>(dst + 16 * h * stride) =
        __builtin_bit_cast(cm_u32x4, __builtin_shufflevector(p0, p1, 0, 1, 2, 3, 4, 5, 6, 7));
  }
}
__device__ __forceinline__ void cm_load_tile(bf16* sw, float* v, const bf16* base, int64_t stride) {
  const int lane = threadIdx.x & 63, half = lane >> 5;
  const int L = lane & 15, G = lane >> 4;
  const bf16* const src = base + (lane >> 2) * stride + 8 * (lane & 3);
  const cm_u32x4 a = *reinterpret_cast<const cm_u32x4*>(src);
  const cm_u32x4 b = *reinterpret_cast<const cm_u32x4*>(src + 16 * stride);
  __builtin_amdgcn_wave_barrier();
  bf16* const w0 = sw + (lane >> 2) * kCmRow + 8 * (lane & 3);
  *reinterpret_cast<cm_u32x2*>(w0) = cm_u32x2{a[0], a[1]};
  *reinterpret_cast<cm_u32x2*>(w0 + 4) = cm_u32x2{a[2], a[3]};
  *reinterpret_cast<cm_u32x2*>(w0 + 16 * kCmRow) = cm_u32x2{b[0], b[1]};
  *reinterpret_cast<cm_u32x2*>(w0 + 16 * kCmRow + 4) = cm_u32x2{b[2], b[3]};
  __builtin_amdgcn_wave_barrier();
#pragma unroll
  for (int g = 0; g < 4; ++g) {
    const s16x4 p = lds_read_tr16(sw + (8 * g + 4 * half + (L >> 2)) * kCmRow + 16 * (G & 1) + 4 * (L & 3));
#pragma unroll
    for (int k = 0; k < 4; ++k) v[4 * g + k] = __uint_as_float((uint32_t)(unsigned short)p[k] << 16);
  }
}

// Column-major ([channel][pitch] pairs) stores of 32-pair x 32-channel tiles
// held in accumulator order: lane l holds pair p0 + (l & 31) and v[4g + r] is
// channel c0 + 8g + 4(l >> 5) + r.  Stored directly, every value is a 2-byte
// store.  The fast path transposes the tile through two MFMAs against
// identity fragments (exact: one product by 1.0 per output) so that lane l
// holds channel c0 + (l & 31) for pairs 8g + 4(l >> 5) .. +3, and writes
// them as 8-byte stores.  Fast requires all 32 pairs of the tile to be real
// and p0 % 4 == 0 (8-byte alignment).
struct CmTile {
  Frag<bf16> id[2];  // k (channels, vals_to_frags order) -> column = channel
  __device__ __forceinline__ CmTile() {
    const int lane = threadIdx.x & 63;
    const int col = lane & 31, half = lane >> 5;
#pragma unroll
    for (int gp = 0; gp < 2; ++gp) {
      float f[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) f[e] = (col == 16 * gp + 8 * (e >> 2) + 4 * half + (e & 3)) ? 1.f : 0.f;
      id[gp].set(f);
    }
  }
  // oz: 0 (an opaque zero in persistent loops, so that the per-lane channel
  // offsets are not hoisted out of them into registers)
  __device__ __forceinline__ void store(bf16* cm, int64_t pitch, int64_t p0, int c0, const float* v, bool fast,
                                        bool lane_valid, int oz = 0) const {
    const int lane = threadIdx.x & 63;
    const int half = lane >> 5, t32 = lane & 31;
    if (fast) {
      Frag<bf16> f[2];
      vals_to_frags<bf16>(f, v);
      f32x16 d = __builtin_amdgcn_mfma_f32_32x32x16_bf16(f[0].v, id[0].v, zero16(), 0, 0, 0);
      d = __builtin_amdgcn_mfma_f32_32x32x16_bf16(f[1].v, id[1].v, d, 0, 0, 0);
      bf16* col = cm + (int64_t)(c0 + t32 + oz) * pitch + p0 + 4 * half;
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const uint2 w = make_uint2(pack_bf16x2(d[4 * g], d[4 * g + 1]), pack_bf16x2(d[4 * g + 2], d[4 * g + 3]));
        *reinterpret_cast<uint2*>(col + 8 * g) = w;
      }
    } else if (lane_valid) {
#pragma unroll
      for (int g = 0; g < 4; ++g)
#pragma unroll
        for (int r = 0; r < 4; ++r)
          cm[(int64_t)(c0 + 8 * g + 4 * half + r + oz) * pitch + p0 + t32] = (bf16)v[4 * g + r];
    }
  }
};

// The same for a 32-pair tile of C = 128 channels in row-half order (lane l
// holds pair p0 + (l & 31) and v[i] is channel 64(l >> 5) + i, i < 64).  Output
// tile s0 = 0, 2, 4, 6 takes k-steps s0 and s0 + 1 (channels 8s .. 8s+7 from the
// lower half-wave, 64 + 8s .. from the upper), so its column c is channel
// 8 s0 + c (c < 16) or 64 + 8 s0 + c - 16.
struct CmTileRH {
  Frag<bf16> id[2];  // k-step s0 + u: k-slot 8h + e -> column 8u + 16h + e
  __device__ __forceinline__ CmTileRH() {
    const int lane = threadIdx.x & 63;
    const int col = lane & 31, half = lane >> 5;
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      float f[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) f[e] = (col == 8 * u + 16 * half + e) ? 1.f : 0.f;
      id[u].set(f);
    }
  }
  __device__ __forceinline__ void store(bf16* cm, int64_t pitch, int64_t p0, const float* v, bool fast,
                                        bool lane_valid, int oz = 0) const {
    const int lane = threadIdx.x & 63;
    const int half = lane >> 5, t32 = lane & 31;
    if (fast) {
#pragma unroll
      for (int s0 = 0; s0 < 8; s0 += 2) {
        Frag<bf16> f0, f1;
        f0.set(v + 8 * s0);
        f1.set(v + 8 * s0 + 8);
        f32x16 d = __builtin_amdgcn_mfma_f32_32x32x16_bf16(f0.v, id[0].v, zero16(), 0, 0, 0);
        d = __builtin_amdgcn_mfma_f32_32x32x16_bf16(f1.v, id[1].v, d, 0, 0, 0);
        const int ch = t32 < 16 ? 8 * s0 + t32 : 64 + 8 * s0 + t32 - 16;
        bf16* col = cm + (int64_t)(ch + oz) * pitch + p0 + 4 * half;
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const uint2 w = make_uint2(pack_bf16x2(d[4 * g], d[4 * g + 1]), pack_bf16x2(d[4 * g + 2], d[4 * g + 3]));
          *reinterpret_cast<uint2*>(col + 8 * g) = w;
        }
      }
    } else if (lane_valid) {
#pragma unroll
      for (int i = 0; i < 64; ++i) cm[(int64_t)(half * 64 + i + oz) * pitch + p0 + t32] = (bf16)v[i];
    }
  }
};

// out = in^T per [Np][Np] plane, 64x64 tiles through LDS.  Np % 64 == 0.
template <typename T>
__global__ __launch_bounds__(256) void transpose_planes_kernel(const T* __restrict__ in,
                                                               T* __restrict__ out, int Np,
                                                               int64_t nplanes) {
  __shared__ T tile[64][65];
  const int t1 = Np / 64;
  const int64_t lin = blockIdx.x;
  const int64_t pl = lin / ((int64_t)t1 * t1);
  const int rem = (int)(lin % ((int64_t)t1 * t1));
  const int i0 = (rem / t1) * 64, j0 = (rem % t1) * 64;
  const int64_t plane = (int64_t)Np * Np;
  const T* src = in + pl * plane;
  T* dst = out + pl * plane;
  const int tx = threadIdx.x & 63, ty = wave_id();
#pragma unroll 4
  for (int r = ty; r < 64; r += 4) tile[r][tx] = src[(int64_t)(i0 + r) * Np + j0 + tx];
  __syncthreads();
#pragma unroll 4
  for (int r = ty; r < 64; r += 4) dst[(int64_t)(j0 + r) * Np + i0 + tx] = tile[tx][r];
}

template <typename T>
inline int launch_transpose_planes(const T* in, T* out, int Np, int64_t nplanes, hipStream_t st) {
  const int64_t blocks = (int64_t)(Np / 64) * (Np / 64) * nplanes;
  GTK_REQUIRE(blocks < (1ll << 31), GTK_EUNSUPPORTED, "transpose grid too large");
  if (blocks == 0) return GTK_OK;
  transpose_planes_kernel<T><<<(unsigned)blocks, 256, 0, st>>>(in, out, Np, nplanes);
  GTK_LAUNCH_CHECK();
  return GTK_OK;
}

// Zero columns [P, pitch) of `rows` CM rows.
template <typename T>
__global__ void zero_tail_kernel(T* __restrict__ base, int64_t rows, int64_t pitch, int64_t P) {
  const int64_t w = pitch - P;
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= rows * w) return;
  base[(idx / w) * pitch + P + idx % w] = cvt<T>(0.f);
}

template <typename T>
inline int launch_zero_tail(T* base, int64_t rows, int64_t pitch, int64_t P, hipStream_t st) {
  const int64_t n = rows * (pitch - P);
  if (n <= 0) return GTK_OK;
  zero_tail_kernel<T><<<(unsigned)((n + 255) / 256), 256, 0, st>>>(base, rows, pitch, P);
  GTK_LAUNCH_CHECK();
  return GTK_OK;
}

// ---------------------------------------------------------------------------
// Weight-gradient product  part[s][m][n] = sum_{p in chunk s} G[m][p] X[n][p]
// G: [M][pitch], X: [Nn][pitch] (CM planes, k = p contiguous).  Block: 128 x TN
// output tile, 4 waves of 64 x TN/2, k staged through LDS in 128-byte rows
// with double buffering (the contraction kernel's scheme).  Chunk s covers
// p in [s*kc, min((s+1)*kc, pitch)), kc a multiple of 64.
// RS: also rs[s][m] = sum_{p in chunk s} G[m][p] (the bias gradients), summed
// from the staged G chunks by the blocks of the first n tile; this replaces a
// separate pass over G.
// ---------------------------------------------------------------------------
template <typename T, int TN, bool RS = false>
__global__ __launch_bounds__(256) void wgrad_kernel(const T* __restrict__ G, const T* __restrict__ X,
                                                    float* __restrict__ part, int M, int Nn,
                                                    int64_t pitch, int64_t kc, int nsplit,
                                                    float* __restrict__ rs) {
  constexpr int BK = 128 / sizeof(T);
  constexpr int PITCH = 144;
  constexpr int ROWS = 128 + TN;
  constexpr int CPT = ROWS * 8 / 256;  // 16-byte chunks per thread per stage
  constexpr int EPC = 16 / sizeof(T);
  constexpr int MBN = TN / 64;         // 32-wide blocks per wave in n
  __shared__ __attribute__((aligned(16))) char smem[2][ROWS * PITCH];

  const int mtiles = M / 128, ntiles = Nn / TN;
  const int64_t lin = blockIdx.x;
  const int s = (int)(lin % nsplit);
  const int mt = (int)((lin / nsplit) % mtiles);
  const int ntl = (int)(lin / ((int64_t)nsplit * mtiles));
  if (ntl >= ntiles) return;
  const int m0 = mt * 128, n0 = ntl * TN;
  const int64_t kbeg = (int64_t)s * kc;
  const int64_t kend = kbeg + kc < pitch ? kbeg + kc : pitch;

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, half = lane >> 5;
  const int wm = (wave >> 1) * 64, wn = (wave & 1) * (TN / 2);
  f32x16 acc[2][MBN];
#pragma unroll
  for (int x = 0; x < 2; ++x)
#pragma unroll
    for (int y = 0; y < MBN; ++y) acc[x][y] = zero16();

  f32x4 rr[CPT];
  // G rows tid/8 + 32u (u < 4) of this thread's chunks: their partial sums
  float rsum[4] = {0.f, 0.f, 0.f, 0.f};
  const bool do_rs = RS && ntl == 0;
  auto gload = [&](int64_t k0) {
#pragma unroll
    for (int u = 0; u < CPT; ++u) {
      const int id = tid + 256 * u;
      const int row = id >> 3, cc = id & 7;
      const T* src = row < 128 ? G + (int64_t)(m0 + row) * pitch : X + (int64_t)(n0 + row - 128) * pitch;
      rr[u] = *reinterpret_cast<const f32x4*>(src + k0 + cc * EPC);
    }
  };
  auto sstore = [&](int buf) {
#pragma unroll
    for (int u = 0; u < CPT; ++u) {
      const int id = tid + 256 * u;
      const int row = id >> 3, cc = id & 7;
      *reinterpret_cast<f32x4*>(&smem[buf][row * PITCH + cc * 16]) = rr[u];
    }
    if (do_rs) {
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const T* e = reinterpret_cast<const T*>(&rr[u]);
#pragma unroll
        for (int k = 0; k < EPC; ++k) rsum[u] += to_f32(e[k]);
      }
    }
  };
  if (kbeg < kend) {
    gload(kbeg);
    sstore(0);
  }
  __syncthreads();
  int cur = 0;
  for (int64_t k0 = kbeg; k0 < kend; k0 += BK) {
    const bool more = k0 + BK < kend;
    if (more) gload(k0 + BK);
#pragma unroll
    for (int kk = 0; kk < BK / 16; ++kk) {
      const int koff = (kk * 16 + half * 8) * (int)sizeof(T);
      Frag<T> fg[2], fx[MBN];
#pragma unroll
      for (int x = 0; x < 2; ++x)
        fg[x].load(reinterpret_cast<const T*>(&smem[cur][(wm + 32 * x + (lane & 31)) * PITCH + koff]));
#pragma unroll
      for (int y = 0; y < MBN; ++y)
        fx[y].load(reinterpret_cast<const T*>(&smem[cur][(128 + wn + 32 * y + (lane & 31)) * PITCH + koff]));
#pragma unroll
      for (int x = 0; x < 2; ++x)
#pragma unroll
        for (int y = 0; y < MBN; ++y) mma(acc[x][y], fx[y], fg[x]);  // rows n, cols m
    }
    if (more) sstore(cur ^ 1);
    __syncthreads();
    cur ^= 1;
  }
  if (do_rs) {
    // the 8 threads of a row (tid % 8) are 8 consecutive lanes
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      float v = rsum[u];
      v += __shfl_xor(v, 1, 64);
      v += __shfl_xor(v, 2, 64);
      v += __shfl_xor(v, 4, 64);
      if ((tid & 7) == 0) rs[(int64_t)s * M + m0 + (tid >> 3) + 32 * u] = v;
    }
  }
  // acc[x][y]: lane holds W[m = m0 + wm + 32x + (l&31)][n = n0 + wn + 32y + 8g + 4h + r]
  float* out = part + (int64_t)s * M * Nn;
#pragma unroll
  for (int x = 0; x < 2; ++x) {
    const int m = m0 + wm + 32 * x + (lane & 31);
#pragma unroll
    for (int y = 0; y < MBN; ++y)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int n = n0 + wn + 32 * y + 8 * g + 4 * half;
        store4(out + (int64_t)m * Nn + n, acc[x][y][4 * g], acc[x][y][4 * g + 1],
               acc[x][y][4 * g + 2], acc[x][y][4 * g + 3]);
      }
  }
}

// bf16 form of wgrad_kernel with the k stages copied straight into a 4-stage
// LDS ring (global_load_lds_dwordx4, three stages in flight, no VGPR
// staging).  The stage is 128 + TN rows of 128 bytes, 16-byte chunk c of row r
// at c ^ ((r ^ (r >> 3)) & 7), so the fragment reads are bank-conflict free;
// copy n of a stage moves rows 8n .. 8n + 7 (1 KiB), wave w the copies
// w, w + 4, ...  RS: the waves of n half 0 add the G fragments they read.
template <int TN, bool RS>
__global__ __launch_bounds__(256) void wgrad_ring_kernel(const bf16* __restrict__ G, const bf16* __restrict__ X,
                                                         float* __restrict__ part, int M, int Nn, int64_t pitch,
                                                         int64_t kc, int nsplit, float* __restrict__ rs) {
  constexpr int BK = 64, NS = 4;
  constexpr int ROWS = 128 + TN;
  constexpr int CPW = ROWS / 8 / 4;  // copies per wave per stage
  constexpr int MBN = TN / 64;       // 32-wide blocks per wave in n
  __shared__ __attribute__((aligned(1024))) char ring[NS][ROWS * 128];

  const int mtiles = M / 128, ntiles = Nn / TN;
  // the m and n tiles of one split are consecutive logical blocks, and each
  // XCD takes a contiguous range of them (the grid is padded to a multiple of
  // 8), so the blocks that read a split's X chunk share that XCD's L2
  const int64_t lin = xcd_remap(blockIdx.x, gridDim.x);
  if (lin >= (int64_t)nsplit * mtiles * ntiles) return;
  const int mt = (int)(lin % mtiles);
  const int ntl = (int)((lin / mtiles) % ntiles);
  const int s = (int)(lin / ((int64_t)mtiles * ntiles));
  const int m0 = mt * 128, n0 = ntl * TN;
  const int64_t kbeg = (int64_t)s * kc;
  const int64_t kend = kbeg + kc < pitch ? kbeg + kc : pitch;
  const int S = kbeg < kend ? (int)((kend - kbeg) / BK) : 0;

  const int tid = threadIdx.x, lane = tid & 63, wave = wave_id(), half = lane >> 5;
  const int wm = (wave >> 1) * 64, wn = (wave & 1) * (TN / 2);
  f32x16 acc[2][MBN];
#pragma unroll
  for (int x = 0; x < 2; ++x)
#pragma unroll
    for (int y = 0; y < MBN; ++y) acc[x][y] = zero16();

  // per-lane byte offsets of copy u (n = wave + 4u): row n*8 + lane/8,
  // physical chunk lane%8 holding logical chunk (lane%8) ^ swz(row)
  uint32_t voff[CPW];
#pragma unroll
  for (int u = 0; u < CPW; ++u) {
    const int n = wave + 4 * u, j = lane >> 3;
    voff[u] = (uint32_t)((j * pitch + 8 * (((lane & 7) ^ (j ^ n)) & 7)) * 2);
  }
  const uint32_t ring_lds = lds_addr(ring);
  auto issue = [&](int st) {
    const int64_t k0 = kbeg + (int64_t)st * BK;
#pragma unroll
    for (int u = 0; u < CPW; ++u) {
      const int n = wave + 4 * u;
      const int row = 8 * n;
      const bf16* base = row < 128 ? G + (int64_t)(m0 + row) * pitch + k0 : X + (int64_t)(n0 + row - 128) * pitch + k0;
      g2lds16_sv(base, voff[u], ring_lds + (uint32_t)((st % NS) * ROWS * 128 + n * 1024));
    }
  };
  auto swz = [](int r) { return (r ^ (r >> 3)) & 7; };
  float rsum[2] = {0.f, 0.f};
  const bool do_rs = RS && ntl == 0 && (wave & 1) == 0;

  for (int st = 0; st < 3 && st < S; ++st) issue(st);
  for (int st = 0; st < S; ++st) {
    // this wave's copies of stage st landed: behind them are those of the
    // (at most two) stages issued after it
    const int later = S - 1 - st < 2 ? S - 1 - st : 2;
    if (later == 2) __builtin_amdgcn_s_waitcnt(vmcnt_imm<2 * CPW>());
    else if (later == 1) __builtin_amdgcn_s_waitcnt(vmcnt_imm<CPW>());
    else __builtin_amdgcn_s_waitcnt(vmcnt_imm<0>());
    barrier_only();  // stage st visible to every wave; stage st - 1 fully read
    if (st + 3 < S) issue(st + 3);
    const char* sb = ring[st % NS];
#pragma unroll
    for (int kk = 0; kk < BK / 16; ++kk) {
      const int lc = kk * 2 + half;  // logical 16-byte chunk
      Frag<bf16> fg[2], fx[MBN];
#pragma unroll
      for (int x = 0; x < 2; ++x) {
        const int r = wm + 32 * x + (lane & 31);
        fg[x].load(reinterpret_cast<const bf16*>(sb + r * 128 + 16 * (lc ^ swz(r))));
      }
#pragma unroll
      for (int y = 0; y < MBN; ++y) {
        const int r = 128 + wn + 32 * y + (lane & 31);
        fx[y].load(reinterpret_cast<const bf16*>(sb + r * 128 + 16 * (lc ^ swz(r))));
      }
#pragma unroll
      for (int x = 0; x < 2; ++x)
#pragma unroll
        for (int y = 0; y < MBN; ++y) mma(acc[x][y], fx[y], fg[x]);  // rows n, cols m
      if (do_rs) {
#pragma unroll
        for (int x = 0; x < 2; ++x)
#pragma unroll
          for (int e = 0; e < 8; ++e) rsum[x] += fg[x].get(e);
      }
    }
  }
  if (do_rs) {
#pragma unroll
    for (int x = 0; x < 2; ++x) {
      const float v = rsum[x] + xor32(rsum[x]);
      if (half == 0) rs[(int64_t)s * M + m0 + wm + 32 * x + (lane & 31)] = v;
    }
  }
  // acc[x][y]: lane holds W[m = m0 + wm + 32x + (l&31)][n = n0 + wn + 32y + 8g + 4h + r]
  float* out = part + (int64_t)s * M * Nn;
#pragma unroll
  for (int x = 0; x < 2; ++x) {
    const int m = m0 + wm + 32 * x + (lane & 31);
#pragma unroll
    for (int y = 0; y < MBN; ++y)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int n = n0 + wn + 32 * y + 8 * g + 4 * half;
        store4(out + (int64_t)m * Nn + n, acc[x][y][4 * g], acc[x][y][4 * g + 1],
               acc[x][y][4 * g + 2], acc[x][y][4 * g + 3]);
      }
  }
}

struct WgradPlan {
  int nsplit;
  int64_t kc;
};

// The product runs on the kernel's tiles: M rounded up to 128 and Nn to 64 or
// a multiple of 128.  Output (m, n) reads only rows m of G and n of X, so the
// extra rows may hold anything: the callers' G and X buffers have at least
// wgrad_m_rows(M) and wgrad_n_rows(Nn) rows of `pitch`, and the outputs of
// the extra rows are never read.
inline int wgrad_m_rows(int M) { return (M + 127) / 128 * 128; }
inline int wgrad_n_rows(int Nn) { return Nn <= 64 ? 64 : (Nn + 127) / 128 * 128; }
// rows of a buffer used as G of one product and X of another
inline int wgrad_rows(int rows) { return wgrad_m_rows(rows); }

// Splits: about one block per CU (MI355X: 256) and never more than that, so
// that no straggler round of a few blocks doubles the launch (515 blocks of
// 2 per CU ran as two rounds of one block's time each); the bf16 ring kernel
// holds one block per CU.
constexpr int kWgradBlocks = 256;
inline WgradPlan wgrad_plan(int M, int64_t pitch) {
  const int mtiles = wgrad_m_rows(M) / 128;
  int64_t ns = kWgradBlocks / mtiles;
  const int64_t maxs = pitch / 64 > 0 ? pitch / 64 : 1;
  if (ns > maxs) ns = maxs;
  if (ns < 1) ns = 1;
  int64_t kc = round_up((pitch + ns - 1) / ns, 64);
  ns = (pitch + kc - 1) / kc;
  return WgradPlan{(int)(ns > 0 ? ns : 1), kc};
}

inline size_t wgrad_part_floats(int M, int Nn, int64_t pitch) {
  return (size_t)wgrad_plan(M, pitch).nsplit * wgrad_m_rows(M) * wgrad_n_rows(Nn);
}
// floats of the row-sum partials rs[nsplit][wgrad_m_rows(M)]
inline size_t wgrad_rowsum_floats(int M, int64_t pitch) {
  return (size_t)wgrad_plan(M, pitch).nsplit * wgrad_m_rows(M);
}

// Row ranges of one product's output, each finished into its own tensor.
struct WgradSegs {
  static constexpr int kMax = 8;
  float* dst[kMax];
  int m0[kMax];
  int rows[kMax];
  int count = 0;
  void add(float* d, int m, int r) {
    if (!d || r == 0) return;
    dst[count] = d;
    m0[count] = m;
    rows[count] = r;
    ++count;
  }
};

// Segment k = blockIdx.y: dst_k[(m - m0_k)][n] = sum_s part[s][m][n] * (gamma ? gamma[n] : 1)
//   + (rowsum && beta ? rowsum[m] * beta[n] : 0),  m in [m0_k, m0_k + rows_k),
// n < Nn, with part laid out as [nsplit][Mp][Np] (the padded product).
// Block: 32 consecutive outputs x 8 chunks of the splits (chunk c takes s = c,
// c + 8, ..., four loads in flight), the 8 partial sums of each output added
// through LDS.
static __global__ __launch_bounds__(256) void wgrad_finish_kernel(
    const float* __restrict__ part, int nsplit, int Mp, int Np, int Nn, WgradSegs segs,
    const float* __restrict__ rowsum, const float* __restrict__ gamma, const float* __restrict__ beta) {
  __shared__ float red[8][32];
  const int k = blockIdx.y;
  const int o = threadIdx.x & 31, ch = threadIdx.x >> 5;
  const int idx = blockIdx.x * 32 + o;
  if (blockIdx.x * 32 >= segs.rows[k] * Nn) return;  // block-uniform
  const bool live = idx < segs.rows[k] * Nn;
  const int m = segs.m0[k] + (live ? idx / Nn : 0), n = live ? idx % Nn : 0;
  float acc = 0.f;
  if (live) {
    const float* src = part + (int64_t)m * Np + n;
    const int64_t step = (int64_t)Mp * Np;
    float a[4] = {0.f, 0.f, 0.f, 0.f};
    int sp = ch;
    for (; sp + 24 < nsplit; sp += 32)
#pragma unroll
      for (int u = 0; u < 4; ++u) a[u] += src[(sp + 8 * u) * step];
    for (; sp < nsplit; sp += 8) a[0] += src[sp * step];
    acc = (a[0] + a[1]) + (a[2] + a[3]);
  }
  red[ch][o] = acc;
  __syncthreads();
  if (ch != 0 || !live) return;
#pragma unroll
  for (int c = 1; c < 8; ++c) acc += red[c][o];
  if (gamma) acc *= gamma[n];
  if (rowsum && beta) acc += rowsum[m] * beta[n];
  segs.dst[k][idx] = acc;
}

inline int launch_wgrad_finish(const float* part, int M, int Nn, int64_t pitch, const WgradSegs& segs,
                               const float* rowsum, const float* gamma, const float* beta, hipStream_t st) {
  if (segs.count == 0) return GTK_OK;
  int most = 0;
  for (int k = 0; k < segs.count; ++k) most = segs.rows[k] > most ? segs.rows[k] : most;
  const int n = most * Nn;
  wgrad_finish_kernel<<<dim3((n + 31) / 32, segs.count), 256, 0, st>>>(
      part, wgrad_plan(M, pitch).nsplit, wgrad_m_rows(M), wgrad_n_rows(Nn), Nn, segs, rowsum, gamma, beta);
  GTK_LAUNCH_CHECK();
  return GTK_OK;
}

inline int launch_wgrad_finish(const float* part, int M, int Nn, int64_t pitch, int m0, int rows,
                               const float* rowsum, const float* gamma, const float* beta,
                               float* dst, hipStream_t st) {
  WgradSegs segs;
  segs.add(dst, m0, rows);
  return launch_wgrad_finish(part, M, Nn, pitch, segs, rowsum, gamma, beta, st);
}

// part[s][m][n] (m < wgrad_m_rows(M), n < wgrad_n_rows(Nn)): split s of
// sum_k G[m][k] X[n][k].  With rs and sums: also sums[m] = sum_k G[m][k] for
// m < M (rs: wgrad_rowsum_floats(M, pitch) floats of partials).
template <typename T>
inline int launch_wgrad(const T* G, const T* X, float* part, int M, int Nn, int64_t pitch,
                        hipStream_t st, float* rs = nullptr, float* sums = nullptr) {
  GTK_REQUIRE(M >= 1 && Nn >= 1, GTK_EUNSUPPORTED, "weight gradient shape %d x %d unsupported", M, Nn);
  const int Mp = wgrad_m_rows(M), Np = wgrad_n_rows(Nn);
  const WgradPlan pl = wgrad_plan(M, pitch);
  const bool with_rs = rs && sums;
  auto go = [&](auto tn, auto r) {
    constexpr int TN = decltype(tn)::value;
    const int64_t blocks = (int64_t)pl.nsplit * (Mp / 128) * (TN == 128 ? Np / 128 : 1);
    if constexpr (sizeof(T) == 2)
      wgrad_ring_kernel<TN, decltype(r)::value><<<(unsigned)((blocks + 7) / 8 * 8), 256, 0, st>>>(
          (const bf16*)G, (const bf16*)X, part, Mp, Np, pitch, pl.kc, pl.nsplit, rs);
    else
      wgrad_kernel<T, TN, decltype(r)::value><<<(unsigned)blocks, 256, 0, st>>>(G, X, part, Mp, Np, pitch,
                                                                               pl.kc, pl.nsplit, rs);
  };
  using I128 = std::integral_constant<int, 128>;
  using I64 = std::integral_constant<int, 64>;
  if (Np % 128 == 0) {
    if (with_rs) go(I128{}, std::true_type{});
    else go(I128{}, std::false_type{});
  } else {
    if (with_rs) go(I64{}, std::true_type{});
    else go(I64{}, std::false_type{});
  }
  GTK_LAUNCH_CHECK();
  if (with_rs) {
    // rs is a product output of one column: the same split reduction
    WgradSegs one;
    one.add(sums, 0, M);
    wgrad_finish_kernel<<<dim3((M + 31) / 32, 1), 256, 0, st>>>(rs, pl.nsplit, Mp, 1, 1, one, nullptr, nullptr,
                                                                nullptr);
    GTK_LAUNCH_CHECK();
  }
  return GTK_OK;
}


// ---------------------------------------------------------------------------
// Row reductions over CM planes: psum[r][s] = sum over segment s of G[r][.],
// pdot[r][s] = the same of G[r][.] * X[r][.] (X may be null).
// ---------------------------------------------------------------------------
constexpr int kRowSegs = 8;

template <typename T, bool DOT>
__global__ __launch_bounds__(256) void rowred_kernel(const T* __restrict__ G, const T* __restrict__ X,
                                                     int rows, int64_t pitch, int64_t P,
                                                     float* __restrict__ psum, float* __restrict__ pdot) {
  __shared__ float red[2][4];
  constexpr int STEP = 8 * 256;  // entries a block reads per pass
  const int nseg = (int)(gridDim.x / rows);
  const int r = blockIdx.x / nseg, s = blockIdx.x % nseg;
  const int64_t seg = ((P + nseg - 1) / nseg + 7) / 8 * 8;
  const int64_t b0 = s * seg;
  const int64_t b1 = b0 + seg < P ? b0 + seg : P;
  const int64_t full = b0 + (b1 > b0 ? (b1 - b0) / 8 * 8 : 0);  // end of the whole 8-entry chunks
  const T* g = G + (int64_t)r * pitch;
  const T* x = DOT ? X + (int64_t)r * pitch : nullptr;
  float a = 0.f, d = 0.f;
  int64_t p = b0 + 8 * threadIdx.x;
  // four independent 16-byte loads in flight a thread (one at a time leaves
  // the reduction bound by load latency at well under the HBM rate)
  for (; p + 3 * STEP < full; p += 4 * STEP) {
    Frag<T> fg[4], fx[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      fg[u].load(g + p + u * STEP);
      if constexpr (DOT) fx[u].load(x + p + u * STEP);
    }
#pragma unroll
    for (int u = 0; u < 4; ++u)
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float v = fg[u].get(e);
        a += v;
        if constexpr (DOT) d += v * fx[u].get(e);
      }
  }
  for (; p < b1; p += STEP) {
    Frag<T> fg, fx;
    fg.load(g + p);  // the row extends to pitch >= P rounded to 8
    if constexpr (DOT) fx.load(x + p);
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const bool in = p + e < b1;
      const float v = in ? fg.get(e) : 0.f;
      a += v;
      if constexpr (DOT) d += v * (in ? fx.get(e) : 0.f);
    }
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    a += __shfl_xor(a, o, 64);
    d += __shfl_xor(d, o, 64);
  }
  const int wave = wave_id();
  if ((threadIdx.x & 63) == 0) {
    red[0][wave] = a;
    red[1][wave] = d;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    psum[(int64_t)r * nseg + s] = red[0][0] + red[0][1] + red[0][2] + red[0][3];
    if (DOT) pdot[(int64_t)r * nseg + s] = red[1][0] + red[1][1] + red[1][2] + red[1][3];
  }
}

// One wave a row: lane l adds segments l, l + 64, ...
static __global__ __launch_bounds__(64) void rowred_finish_kernel(const float* __restrict__ ps,
                                                                 const float* __restrict__ pd, int rows, int nseg,
                                                                 float* __restrict__ sums, float* __restrict__ dots) {
  const int r = blockIdx.x, l = threadIdx.x;
  float a = 0.f, d = 0.f;
  for (int s = l; s < nseg; s += 64) {
    a += ps[(int64_t)r * nseg + s];
    if (dots) d += pd[(int64_t)r * nseg + s];
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    a += __shfl_xor(a, o, 64);
    d += __shfl_xor(d, o, 64);
  }
  if (l == 0) {
    sums[r] = a;
    if (dots) dots[r] = d;
  }
}

// Segments a row is split into: kRowSegs, or more for few rows (so that the
// launch still has about 1024 blocks); rows x segments <= max(8 rows, 1024),
// which bounds the partials in tmp (2 x that many floats).
inline int rowred_segs(int rows) { return rows >= 128 ? kRowSegs : 1024 / rows; }

// sums[r] (and dots[r] when X is given) for rows [0, rows) of G; tmp holds
// 2 * rows * rowred_segs(rows) floats of partials.
template <typename T>
inline int launch_rowred(const T* G, const T* X, int rows, int64_t pitch, int64_t P, float* tmp,
                         float* sums, float* dots, hipStream_t st) {
  if (rows == 0) return GTK_OK;
  const int nseg = rowred_segs(rows);
  float* ps = tmp;
  float* pd = tmp + (size_t)rows * nseg;
  if (X) rowred_kernel<T, true><<<rows * nseg, 256, 0, st>>>(G, X, rows, pitch, P, ps, pd);
  else rowred_kernel<T, false><<<rows * nseg, 256, 0, st>>>(G, nullptr, rows, pitch, P, ps, nullptr);
  GTK_LAUNCH_CHECK();
  rowred_finish_kernel<<<rows, 64, 0, st>>>(ps, pd, rows, nseg, sums, X ? dots : nullptr);
  GTK_LAUNCH_CHECK();
  return GTK_OK;
}

static __global__ void copy_f32_kernel(float* __restrict__ dst, const float* __restrict__ src, int n) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) dst[i] = src[i];
}
inline int launch_copy_f32(float* dst, const float* src, int n, hipStream_t st) {
  if (!dst || n == 0) return GTK_OK;
  copy_f32_kernel<<<(n + 255) / 256, 256, 0, st>>>(dst, src, n);
  GTK_LAUNCH_CHECK();
  return GTK_OK;
}

// Several small fp32 copies in one launch (block y = copy k).
struct CopyList {
  static constexpr int kMax = 8;
  float* dst[kMax];
  const float* src[kMax];
  int n[kMax];
  int count = 0;
  void add(float* d, const float* s, int len) {
    if (!d || len == 0) return;
    dst[count] = d;
    src[count] = s;
    n[count] = len;
    ++count;
  }
};
static __global__ void copy_list_kernel(CopyList l) {
  const int k = blockIdx.y;
  for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < l.n[k]; i += gridDim.x * blockDim.x)
    l.dst[k][i] = l.src[k][i];
}
inline int launch_copy_list(const CopyList& l, hipStream_t st) {
  if (l.count == 0) return GTK_OK;
  GTK_REQUIRE(l.count <= CopyList::kMax, GTK_EINVAL, "copy list overflow");
  copy_list_kernel<<<dim3(1, l.count), 256, 0, st>>>(l);
  GTK_LAUNCH_CHECK();
  return GTK_OK;
}

}  // namespace gtk
