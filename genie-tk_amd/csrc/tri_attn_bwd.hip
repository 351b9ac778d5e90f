// Backward of triangle attention (starting / ending node).
//
// The reference trains through torch autograd of its PyTorch path
// (triangle_attention.py:100-143 with Attention.forward, primitives.py:114-178);
// this is the same chain rule on gfx950 kernels.  Everything runs in the
// attention orientation (rows r, positions j; the ending node reads x, the
// mask and dL/dy transposed and writes dL/dx transposed).  Forward activations
// are recomputed from x:
//
//  proj   LN(x), q, k, v (position-major and d-major copies), the gate
//         sigmoid, the triangle bias and the key mask of every row.
//  fwd    attention forward per (row, head, 32 queries) with an online
//         softmax: O, the running max m and 1/l per query.
//  epi    dgo = dy W_o, dO = dgo * gate, dg_pre = dgo * O * gate (1 - gate),
//         D = sum_d dO O per (query, head).
//  dkdv   per (row, head, 32 keys): over all queries, P = exp(S - m) / l,
//         dP = dO V^T, dS = P (dP - D); dV = P^T dO, dK = scale dS^T Q.
//  dq     per (row, head, 32 queries): dQ = scale dS K over all keys.
//  dbias  per (head, 32 queries, 32 keys): dB = sum over rows of dS.
//  pro    dxn = dq W_q + dk W_k + dv W_v + dg_pre W_g + dB W_b, LayerNorm
//         backward -> dx; the per-pair operands of the weight gradients.
//  then   split-K weight-gradient products and row sums (grad_util.hpp).
//
// Scores: S = scale q.k + bias for a valid key, exactly -1e9 for a masked key
// (the fp32 reference's qk + (-1e9) + tri rounds to -1e9) and -inf for the
// positions past N.  A row whose keys are all masked is uniform over its N
// keys, and its dS still flows into q, k and the bias: torch autograd of the
// reference differentiates qk + mask_bias + tri term by term.  m and 1/l are
// kept separately (not m + log l): for such a row m = -1e9 and fp32 cannot
// hold -1e9 + log l.
#include <algorithm>
#include <cstdlib>
#include <cmath>
#include <type_traits>

#include "capi_util.hpp"
#include "common.hpp"
#include "grad_util.hpp"
#include "pack.hpp"

namespace gtk {

constexpr int AD = 32;            // head dimension
constexpr float kMaskScore = -1e9f;

template <typename T> struct AttnBwdW {
  T *w_q, *w_k, *w_v, *w_g, *w_b;      // natural units, LayerNorm weight folded in
  float *b_q, *b_k, *b_v, *b_g, *b_b;  // W beta (+ the Linear's bias)
  T *wt_q, *wt_k, *wt_v, *wt_g;        // W^T (unfolded), accumulator order: dxn = d W
  T* wt_o;                             // W_o^T, fragment order: dgo = dy W_o
  float* wb_raw;                       // W_b [H][C], fp32
  float *ln_w, *ln_b;
};

template <typename T> struct AttnBwdBufs {
  T *qr, *qt, *kr, *kt, *vr, *vt;  // [B][N][H][np][32] and [B][N][H][32][np]
  T *o, *dor, *dot, *dq, *dk, *dv; // o, dO, dq, dk, dv position-major; dot d-major
  T* gt;                           // gate sigmoid [B][N][np][CH]
  T* bias;                         // triangle bias [B][H][N][N]
  float *biasT, *biasS;            // bias / scale, fp32, fragment order (bias_frag_elem)
  float* kmask;                    // [B][N][np]: 1 valid key, 0 masked
  float *mrow, *linv, *dd;         // [B][N][H][np]
  float* db;                       // dL/dbias [B][H][N][N]
  float* dbp;                      // dL/dbias partial sums per row chunk (bf16 path, np <= 512)
  T *cm_stack, *cm_xh, *cm_dxn, *cm_dy, *cm_go, *cm_dtri;
  int64_t pitch;
};

// Two k-steps over d = 32 of a 32x32 product: rows from `a`, columns from `b`,
// both operands position-major [pos][32] (lane = position, 8 consecutive d).
template <typename T>
__device__ __forceinline__ f32x16 qk_tile(const T* a_rows, const T* b_rows) {
  const int lane = threadIdx.x & 63;
  const int t32 = lane & 31, half = lane >> 5;
  Frag<T> fa, fb;
  f32x16 acc = zero16();
#pragma unroll
  for (int s = 0; s < 2; ++s) {
    fa.load(a_rows + t32 * AD + 16 * s + 8 * half);
    fb.load(b_rows + t32 * AD + 16 * s + 8 * half);
    mma(acc, fa, fb);
  }
  return acc;
}

// Operand with lane = d and k = 32 positions in accumulator order, from a
// d-major [32][np] block at position p0: chunk gp holds positions
// p0 + 16gp + 8(e>>2) + 4h + (e&3).
template <typename T>
__device__ __forceinline__ void dmajor_frags(Frag<T>* f, const T* base, int64_t np, int p0) {
  const int lane = threadIdx.x & 63;
  const int t32 = lane & 31, half = lane >> 5;
  const T* row = base + (int64_t)t32 * np + p0 + 4 * half;
#pragma unroll
  for (int gp = 0; gp < 2; ++gp) {
    const f32x4 lo = load4f(row + 16 * gp);
    const f32x4 hi = load4f(row + 16 * gp + 8);
    float v[8] = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
    f[gp].set(v);
  }
}

__device__ __forceinline__ float score_of(float acc, float scale, float bias, float km, bool exists) {
  return exists ? (km > 0.5f ? scale * acc + bias : kMaskScore) : -INFINITY;
}

// Triangle-bias copies of the (row, head) kernels: fp32 tiles of 32 x 32 in
// the accumulator order of the score tile that consumes them, 4 KiB each.
// Element (h, a, k) of an orientation whose lanes are positions a and whose
// registers are positions k (register 4g + rr of lane hh*32 + a%32 <-> k%32 =
// 8g + 4hh + rr), at float index
//   (((h * nt + a/32) * nt + k/32) * 4 + g) * 64 + hh*32 + a%32) * 4 + rr.
// biasT has lanes = queries, registers = keys (S^T = K Q^T); biasS has lanes =
// keys, registers = queries (S = Q K^T).  Both hold bias / scale, so the score
// MFMA accumulates q.k onto them directly.
__host__ __device__ __forceinline__ int64_t bias_frag_elem(int h, int a, int k, int np) {
  const int nt = np / 32;
  const int64_t tile = ((int64_t)h * nt + (a >> 5)) * nt + (k >> 5);
  return (((tile * 4 + ((k & 31) >> 3)) * 64 + ((k >> 2) & 1) * 32 + (a & 31)) << 2) + (k & 3);
}

// ---------------------------------------------------------------------------
// proj: one 32-position tile of one attention row per wave
// ---------------------------------------------------------------------------
template <typename T, int C, int H>
__global__ __launch_bounds__(256) void attn_bwd_proj_kernel(const T* __restrict__ x,
                                                            const float* __restrict__ mask,
                                                            AttnBwdW<T> w, AttnBwdBufs<T> bf,
                                                            int B, int N, int np, int starting,
                                                            float eps, float inv_scale, int dmajor) {
  constexpr int CH = H * AD;
  const int lane = threadIdx.x & 63, half = lane >> 5, t32 = lane & 31;
  const int jtiles = np / 32;
  const int64_t tile = (int64_t)blockIdx.x * 4 + wave_id();
  if (tile >= (int64_t)B * N * jtiles) return;
  const int jt = (int)(tile % jtiles);
  const int r = (int)((tile / jtiles) % N);
  const int b = (int)(tile / ((int64_t)jtiles * N));
  const int j = jt * 32 + t32;
  const bool valid = j < N;
  const int64_t xp = valid ? ((int64_t)b * N + (starting ? r : j)) * N + (starting ? j : r) : 0;

  RowHalf<C> rh;
  load_row_half<T, C>(rh, x + xp * C, valid);
  const f32x2 st = row_stats<C>(rh, eps);
  Frag<T> xf[C / 16];
  ln_to_frags<T, C>(xf, rh, st);

  const T* wk[3] = {w.w_q, w.w_k, w.w_v};
  const float* bk[3] = {w.b_q, w.b_k, w.b_v};
  T* dr[3] = {bf.qr, bf.kr, bf.vr};
  T* dt[3] = {bf.qt, bf.kt, bf.vt};
#pragma unroll 1
  for (int kind = 0; kind < 3; ++kind) {
#pragma unroll 1
    for (int h = 0; h < H; ++h) {
      const f32x16 acc = row_gemm_tile<T, C, true>(xf, wk[kind], h);
      const int64_t rh_ = ((int64_t)b * N + r) * H + h;
      T* rowm = dr[kind] + (rh_ * np + j) * AD;
      T* dmaj = dt[kind] + rh_ * AD * np + j;
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int d0 = 8 * g + 4 * half;
        float v[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) v[q] = valid ? acc[4 * g + q] + bk[kind][h * AD + d0 + q] : 0.f;
        store4(rowm + d0, v[0], v[1], v[2], v[3]);
        if (dmajor) {
#pragma unroll
          for (int q = 0; q < 4; ++q) dmaj[(int64_t)(d0 + q) * np] = cvt<T>(v[q]);
        }
      }
    }
  }
#pragma unroll 1
  for (int h = 0; h < H; ++h) {
    const f32x16 acc = row_gemm_tile<T, C, true>(xf, w.w_g, h);
    T* gp = bf.gt + (((int64_t)b * N + r) * np + j) * CH + h * AD;
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const int d0 = 8 * g + 4 * half;
      float v[4];
#pragma unroll
      for (int q = 0; q < 4; ++q) v[q] = sigmoidf_(acc[4 * g + q] + w.b_g[h * AD + d0 + q]);
      store4(gp + d0, v[0], v[1], v[2], v[3]);
    }
  }
  {
    // triangle bias: outputs 0..H-1 sit in lanes of half 0, acc[0..H-1]
    const f32x16 acc = row_gemm_tile<T, C, true>(xf, w.w_b, 0);
    if (valid && half == 0) {
      float* bT = bf.biasT + (int64_t)b * H * np * np;
      float* bS = bf.biasS + (int64_t)b * H * np * np;
#pragma unroll
      for (int h = 0; h < H; ++h) {
        const T bv = cvt<T>(acc[h] + w.b_b[h]);
        bf.bias[(((int64_t)b * H + h) * N + r) * N + j] = bv;
        const float bs = to_f32(bv) * inv_scale;  // query r, key j
        bT[bias_frag_elem(h, r, j, np)] = bs;
        bS[bias_frag_elem(h, j, r, np)] = bs;
      }
    }
  }
  // 1 for a valid key (mask == 1: no bias); 0 for a masked key, whose bias
  // 1e9 * (mask - 1) <= -60 takes it out of any row with a valid key
  if (half == 0) bf.kmask[((int64_t)b * N + r) * np + j] = valid && (!mask || mask[xp] == 1.f) ? 1.f : 0.f;
}

// ---------------------------------------------------------------------------
// proj, bf16 (position-major outputs only): the same products as
// attn_bwd_proj_kernel in persistent blocks of NW waves with W_q, W_k, W_v, W_g,
// W_b (c_h x c_in each, 136 KiB at c_in = 128) and their biases in LDS; the
// kernel above reads 136 KiB of weight fragments from L2 per 32-position tile.
// ---------------------------------------------------------------------------
template <int C, int H, int NW>
__global__ __launch_bounds__(64 * NW) void attn_bwd_proj_lds_kernel(const bf16* __restrict__ x,
                                                                const float* __restrict__ mask,
                                                                AttnBwdW<bf16> w, AttnBwdBufs<bf16> bf, int B,
                                                                int N, int np, int starting, float eps,
                                                                float inv_scale, int64_t ntiles) {
  constexpr int CH = H * AD;
  constexpr int PW = C * CH;   // elements of one packed projection
  constexpr int PB = 32 * C;   // the triangle-bias projection (H outputs padded to 32)
  __shared__ __attribute__((aligned(1024))) bf16 wl[4 * PW + PB];
  __shared__ __attribute__((aligned(16))) float bl[4 * CH + 32];
  copy_to_lds_async(wl, w.w_q, PW * 2);
  copy_to_lds_async(wl + PW, w.w_k, PW * 2);
  copy_to_lds_async(wl + 2 * PW, w.w_v, PW * 2);
  copy_to_lds_async(wl + 3 * PW, w.w_g, PW * 2);
  copy_to_lds_async(wl + 4 * PW, w.w_b, PB * 2);
  for (int t = threadIdx.x; t < CH; t += blockDim.x) {
    bl[t] = w.b_q[t];
    bl[CH + t] = w.b_k[t];
    bl[2 * CH + t] = w.b_v[t];
    bl[3 * CH + t] = w.b_g[t];
  }
  if (threadIdx.x < H) bl[4 * CH + threadIdx.x] = w.b_b[threadIdx.x];
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();

  const int lane = threadIdx.x & 63, half = lane >> 5, t32 = lane & 31;
  const int wave = wave_id();
  const int jtiles = np / 32;
  bf16* const dr[3] = {bf.qr, bf.kr, bf.vr};
  for (int64_t tile = (int64_t)blockIdx.x * NW + wave; tile < ntiles; tile += (int64_t)gridDim.x * NW) {
    const int jt = (int)(tile % jtiles);
    const int r = (int)((tile / jtiles) % N);
    const int b = (int)(tile / ((int64_t)jtiles * N));
    const int j = jt * 32 + t32;
    const bool valid = j < N;
    const int64_t xp = valid ? ((int64_t)b * N + (starting ? r : j)) * N + (starting ? j : r) : 0;
    // per-tile LDS reads of the biases through an opaque index (hoisted out of
    // the tile loop they would stay in registers)
    const int oz = opaque_zero();

    Frag<bf16> xf[C / 16];
    {
      RowHalf<C> rh;
      load_row_half<bf16, C>(rh, x + xp * C, valid);
      const f32x2 st = row_stats<C>(rh, eps);
      ln_to_frags<bf16, C>(xf, rh, st);
    }
    auto gemm = [&](const bf16* wp, int nt) {
      f32x16 acc = zero16();
#pragma unroll
      for (int ks = 0; ks < C / 16; ++ks) {
        Frag<bf16> wf;
        load_wfrag_lds(wf, wp, nt, ks, C / 16);
        mma(acc, wf, xf[ks]);
      }
      return acc;
    };
#pragma unroll 1
    for (int kind = 0; kind < 4; ++kind) {
#pragma unroll 1
      for (int h = 0; h < H; ++h) {
        const f32x16 acc = gemm(wl + kind * PW, h);
        const float* bk = bl + kind * CH + h * AD + oz;
        bf16* const dst = kind < 3 ? dr[kind] + ((((int64_t)b * N + r) * H + h) * np + j) * AD
                                   : bf.gt + (((int64_t)b * N + r) * np + j) * CH + h * AD;
        // lane (t32, half) holds channels 8g + 4 half .. +3 (g = 0..3) of
        // position t32; the half-waves trade quads (v_permlane32_swap) so that
        // the lower half holds channels 0-7 and 16-23, the upper 8-15 and
        // 24-31: two 16-byte stores a lane instead of four 8-byte ones
        uint32_t pk[4][2];
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const int d0 = 8 * g + 4 * half;
          const f32x4 bv = *reinterpret_cast<const f32x4*>(bk + d0);
          float v[4];
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            const float u = acc[4 * g + q] + bv[q];
            v[q] = kind < 3 ? (valid ? u : 0.f) : sigmoidf_(u);
          }
          pk[g][0] = pack_bf16x2(v[0], v[1]);
          pk[g][1] = pack_bf16x2(v[2], v[3]);
        }
#pragma unroll
        for (int p2 = 0; p2 < 2; ++p2) {  // channel groups 2 p2 (lower) and 2 p2 + 1 (upper)
          const auto s0 = __builtin_amdgcn_permlane32_swap(pk[2 * p2][0], pk[2 * p2 + 1][0], false, false);
          const auto s1 = __builtin_amdgcn_permlane32_swap(pk[2 * p2][1], pk[2 * p2 + 1][1], false, false);
          // lower: own quad of group 2 p2, then the upper's; upper: the
          // lower's quad of group 2 p2 + 1, then its own
          const uint4 c = half ? make_uint4(s0[0], s1[0], pk[2 * p2 + 1][0], pk[2 * p2 + 1][1])
                               : make_uint4(pk[2 * p2][0], pk[2 * p2][1], s0[1], s1[1]);
          *reinterpret_cast<uint4*>(dst + 16 * p2 + 8 * half) = c;
        }
      }
    }
    {
      // triangle bias: outputs 0..H-1 sit in lanes of half 0, acc[0..H-1]
      const f32x16 acc = gemm(wl + 4 * PW, 0);
      if (valid && half == 0) {
        float* bT = bf.biasT + (int64_t)b * H * np * np;
        float* bS = bf.biasS + (int64_t)b * H * np * np;
#pragma unroll
        for (int h = 0; h < H; ++h) {
          const bf16 bv = cvt<bf16>(acc[h] + bl[4 * CH + h + oz]);
          bf.bias[(((int64_t)b * H + h) * N + r) * N + j] = bv;
          const float bs = to_f32(bv) * inv_scale;  // query r, key j
          bT[bias_frag_elem(h, r, j, np)] = bs;
          bS[bias_frag_elem(h, j, r, np)] = bs;
        }
      }
    }
    // 1 for a valid key (mask == 1: no bias); 0 for a masked key
    if (half == 0) bf.kmask[((int64_t)b * N + r) * np + j] = valid && (!mask || mask[xp] == 1.f) ? 1.f : 0.f;
  }
}

// ---------------------------------------------------------------------------
// fwd: O, m, 1/l per (row, head, 32 queries); lane = query
// ---------------------------------------------------------------------------
template <typename T, int H>
__global__ __launch_bounds__(256) void attn_bwd_fwd_kernel(AttnBwdBufs<T> bf, int B, int N, int np,
                                                           float scale) {
  const int lane = threadIdx.x & 63, half = lane >> 5, t32 = lane & 31;
  const int qtiles = np / 32;
  const int64_t tile = (int64_t)blockIdx.x * 4 + wave_id();
  if (tile >= (int64_t)B * N * H * qtiles) return;
  const int qt = (int)(tile % qtiles);
  const int64_t rh = tile / qtiles;  // (b*N + r)*H + h
  const int h = (int)(rh % H);
  const int64_t br = rh / H;         // b*N + r
  const int b = (int)(br / N);
  const int q = qt * 32 + t32;
  const T* Q = bf.qr + rh * np * AD;
  const T* K = bf.kr + rh * np * AD;
  const T* VT = bf.vt + rh * AD * np;
  const T* Bh = bf.bias + ((int64_t)b * H + h) * N * N;
  const float* km = bf.kmask + br * np;

  float m = -INFINITY, l = 0.f;
  f32x16 oacc = zero16();
  for (int kt = 0; kt < qtiles; ++kt) {
    const f32x16 acc = qk_tile<T>(K + (int64_t)kt * 32 * AD, Q + (int64_t)qt * 32 * AD);
    float s[16];
    float mx = -INFINITY;
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const int k0 = kt * 32 + 8 * g + 4 * half;
      const f32x4 k4 = *reinterpret_cast<const f32x4*>(km + k0);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int key = k0 + e;
        const float bv = (q < N && key < N) ? to_f32(Bh[(int64_t)q * N + key]) : 0.f;
        s[4 * g + e] = score_of(acc[4 * g + e], scale, bv, k4[e], key < N);
        mx = fmaxf(mx, s[4 * g + e]);
      }
    }
    mx = fmaxf(mx, xor32(mx));
    const float mn = fmaxf(m, mx);
    const float alpha = __expf(m - mn);
    float ps = 0.f;
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      s[e] = __expf(s[e] - mn);
      ps += s[e];
    }
    ps += xor32(ps);
    l = l * alpha + ps;
    m = mn;
#pragma unroll
    for (int e = 0; e < 16; ++e) oacc[e] *= alpha;
    Frag<T> fp[2], fv[2];
    vals_to_frags<T>(fp, s);
    dmajor_frags<T>(fv, VT, np, kt * 32);
    mma(oacc, fv[0], fp[0]);
    mma(oacc, fv[1], fp[1]);
  }
  const float li = 1.0f / l;
  T* O = bf.o + (rh * np + q) * AD;
#pragma unroll
  for (int g = 0; g < 4; ++g)
    store4(O + 8 * g + 4 * half, oacc[4 * g] * li, oacc[4 * g + 1] * li, oacc[4 * g + 2] * li,
           oacc[4 * g + 3] * li);
  if (half == 0) {
    bf.mrow[rh * np + q] = m;
    bf.linv[rh * np + q] = li;
  }
}

// ---------------------------------------------------------------------------
// epi: dgo = dy W_o, dO, dg_pre, D; per 32-position tile of one row
// ---------------------------------------------------------------------------
// Row store of one position from the accumulator layout: value 4g + r of
// lane (t32, half) is channel 8g + 4 half + r of the position; the half-waves
// trade channel quads (v_permlane32_swap) so that each lane stores two
// 16-byte pieces of 8 consecutive channels (the lower half channels 0-7 and
// 16-23, the upper 8-15 and 24-31) instead of four 8-byte ones.  Every lane
// of the wave must take part.
__device__ __forceinline__ void store_row32_bf16(bf16* row, const float* v) {
  const int half = (threadIdx.x & 63) >> 5;
  uint32_t pk[4][2];
#pragma unroll
  for (int g = 0; g < 4; ++g) {
    pk[g][0] = pack_bf16x2(v[4 * g], v[4 * g + 1]);
    pk[g][1] = pack_bf16x2(v[4 * g + 2], v[4 * g + 3]);
  }
#pragma unroll
  for (int p2 = 0; p2 < 2; ++p2) {
    const auto s0 = __builtin_amdgcn_permlane32_swap(pk[2 * p2][0], pk[2 * p2 + 1][0], false, false);
    const auto s1 = __builtin_amdgcn_permlane32_swap(pk[2 * p2][1], pk[2 * p2 + 1][1], false, false);
    const uint4 c = half ? make_uint4(s0[0], s1[0], pk[2 * p2 + 1][0], pk[2 * p2 + 1][1])
                         : make_uint4(pk[2 * p2][0], pk[2 * p2][1], s0[1], s1[1]);
    *reinterpret_cast<uint4*>(row + 16 * p2 + 8 * half) = c;
  }
}

template <typename T, int C, int H>
__global__ __launch_bounds__(256) void attn_bwd_epi_kernel(const T* __restrict__ dy, AttnBwdW<T> w,
                                                           AttnBwdBufs<T> bf, int B, int N, int np,
                                                           int starting, int dmajor) {
  constexpr int CH = H * AD;
  const int lane = threadIdx.x & 63, half = lane >> 5, t32 = lane & 31;
  const int jtiles = np / 32;
  const int64_t tile = (int64_t)blockIdx.x * 4 + wave_id();
  if (tile >= (int64_t)B * N * jtiles) return;
  const int jt = (int)(tile % jtiles);
  const int r = (int)((tile / jtiles) % N);
  const int b = (int)(tile / ((int64_t)jtiles * N));
  const int j = jt * 32 + t32;
  const bool valid = j < N;
  const int64_t xp = valid ? ((int64_t)b * N + (starting ? r : j)) * N + (starting ? j : r) : 0;
  const int64_t p = ((int64_t)b * N + r) * N + j;  // pair index, attention orientation
  const int64_t pitch = bf.pitch;
  const int64_t p0 = ((int64_t)b * N + r) * N + jt * 32;
  const bool fast = std::is_same<T, bf16>::value && jt * 32 + 32 <= N && N % 4 == 0;

  RowHalf<C> dh;
  load_row_half<T, C>(dh, dy + xp * C, valid);
  Frag<T> fdy[C / 16];
#pragma unroll
  for (int ch = 0; ch < C / 16; ++ch) fdy[ch].set(&dh.v[ch * 8]);
  if constexpr (std::is_same<T, bf16>::value && C == 128) {
    const CmTileRH cmr;  // whole transposed tiles of the lane's row half
    cmr.store(bf.cm_dy, pitch, p0, dh.v, fast, valid);
  } else if (valid) {
#pragma unroll
    for (int i = 0; i < C / 2; ++i) bf.cm_dy[(int64_t)(half * (C / 2) + i) * pitch + p] = cvt<T>(dh.v[i]);
  }
  T* cm_dg = bf.cm_stack + (int64_t)3 * CH * pitch;
  const CmTile cmt;
#pragma unroll 1
  for (int h = 0; h < H; ++h) {
    const f32x16 dog = row_gemm_tile<T, C, true>(fdy, w.wt_o, h);
    const int64_t rh = ((int64_t)b * N + r) * H + h;
    const T* O = bf.o + (rh * np + j) * AD;
    const T* G = bf.gt + (((int64_t)b * N + r) * np + j) * CH + h * AD;
    T* dor = bf.dor + (rh * np + j) * AD;
    T* dot = bf.dot + rh * AD * np + j;
    float dsum = 0.f;
    float vdg[16], vgo[16];
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const int d0 = 8 * g + 4 * half;
      const f32x4 o4 = load4f(O + d0);
      const f32x4 g4 = load4f(G + d0);
      float dov[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float dg = dog[4 * g + e];
        dov[e] = valid ? dg * g4[e] : 0.f;
        dsum += dov[e] * o4[e];
        vdg[4 * g + e] = dg * o4[e] * g4[e] * (1.f - g4[e]);
        vgo[4 * g + e] = o4[e] * g4[e];
        if constexpr (!std::is_same<T, bf16>::value) {
          if (valid) {
            const int64_t o = (int64_t)(h * AD + d0 + e) * pitch + p;
            cm_dg[o] = cvt<T>(vdg[4 * g + e]);
            bf.cm_go[o] = cvt<T>(vgo[4 * g + e]);
          }
        }
        if (dmajor) dot[(int64_t)(d0 + e) * np] = cvt<T>(dov[e]);
      }
      store4(dor + d0, dov[0], dov[1], dov[2], dov[3]);
    }
    if constexpr (std::is_same<T, bf16>::value) {
      cmt.store(cm_dg, pitch, p0, h * AD, vdg, fast, valid);
      cmt.store(bf.cm_go, pitch, p0, h * AD, vgo, fast, valid);
    }
    dsum += xor32(dsum);
    if (half == 0) bf.dd[rh * np + j] = dsum;
  }
}

// ---------------------------------------------------------------------------
// dkdv: per (row, head, 32 keys); lane = key
// ---------------------------------------------------------------------------
template <typename T, int H>
__global__ __launch_bounds__(256) void attn_bwd_dkdv_kernel(AttnBwdBufs<T> bf, int B, int N, int np,
                                                            float scale) {
  const int lane = threadIdx.x & 63, half = lane >> 5, t32 = lane & 31;
  const int tiles1 = np / 32;
  const int64_t tile = (int64_t)blockIdx.x * 4 + wave_id();
  if (tile >= (int64_t)B * N * H * tiles1) return;
  const int kt = (int)(tile % tiles1);
  const int64_t rh = tile / tiles1;
  const int h = (int)(rh % H);
  const int64_t br = rh / H;
  const int b = (int)(br / N);
  const int key = kt * 32 + t32;
  const bool kexists = key < N;
  const float km = bf.kmask[br * np + key];
  const T* Q = bf.qr + rh * np * AD;
  const T* QT = bf.qt + rh * AD * np;
  const T* K = bf.kr + rh * np * AD + (int64_t)kt * 32 * AD;
  const T* V = bf.vr + rh * np * AD + (int64_t)kt * 32 * AD;
  const T* DO = bf.dor + rh * np * AD;
  const T* DOT = bf.dot + rh * AD * np;
  const T* Bh = bf.bias + ((int64_t)b * H + h) * N * N;
  const float* mr = bf.mrow + rh * np;
  const float* lr = bf.linv + rh * np;
  const float* dr = bf.dd + rh * np;

  f32x16 dk = zero16(), dv = zero16();
  for (int qt = 0; qt < tiles1; ++qt) {
    const f32x16 sa = qk_tile<T>(Q + (int64_t)qt * 32 * AD, K);   // [q][key]: lane = key
    const f32x16 pa = qk_tile<T>(DO + (int64_t)qt * 32 * AD, V);  // dP
    float pv[16], ds[16];
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const int q0 = qt * 32 + 8 * g + 4 * half;
      const f32x4 m4 = *reinterpret_cast<const f32x4*>(mr + q0);
      const f32x4 l4 = *reinterpret_cast<const f32x4*>(lr + q0);
      const f32x4 d4 = *reinterpret_cast<const f32x4*>(dr + q0);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int q = q0 + e;
        const float bv = (q < N && kexists) ? to_f32(Bh[(int64_t)q * N + key]) : 0.f;
        const float s = score_of(sa[4 * g + e], scale, bv, km, kexists);
        const float pr = __expf(s - m4[e]) * l4[e];
        pv[4 * g + e] = pr;
        ds[4 * g + e] = pr * (pa[4 * g + e] - d4[e]);
      }
    }
    Frag<T> fp[2], fs[2], fa[2];
    vals_to_frags<T>(fp, pv);
    vals_to_frags<T>(fs, ds);
    dmajor_frags<T>(fa, DOT, np, qt * 32);
    mma(dv, fa[0], fp[0]);
    mma(dv, fa[1], fp[1]);
    dmajor_frags<T>(fa, QT, np, qt * 32);
    mma(dk, fa[0], fs[0]);
    mma(dk, fa[1], fs[1]);
  }
  T* dko = bf.dk + (rh * np + key) * AD;
  T* dvo = bf.dv + (rh * np + key) * AD;
#pragma unroll
  for (int g = 0; g < 4; ++g) {
    const int d0 = 8 * g + 4 * half;
    store4(dko + d0, scale * dk[4 * g], scale * dk[4 * g + 1], scale * dk[4 * g + 2], scale * dk[4 * g + 3]);
    store4(dvo + d0, dv[4 * g], dv[4 * g + 1], dv[4 * g + 2], dv[4 * g + 3]);
  }
}

// ---------------------------------------------------------------------------
// dq: per (row, head, 32 queries); lane = query
// ---------------------------------------------------------------------------
template <typename T, int H>
__global__ __launch_bounds__(256) void attn_bwd_dq_kernel(AttnBwdBufs<T> bf, int B, int N, int np,
                                                          float scale) {
  const int lane = threadIdx.x & 63, half = lane >> 5, t32 = lane & 31;
  const int tiles1 = np / 32;
  const int64_t tile = (int64_t)blockIdx.x * 4 + wave_id();
  if (tile >= (int64_t)B * N * H * tiles1) return;
  const int qt = (int)(tile % tiles1);
  const int64_t rh = tile / tiles1;
  const int h = (int)(rh % H);
  const int64_t br = rh / H;
  const int b = (int)(br / N);
  const int q = qt * 32 + t32;
  const T* Q = bf.qr + rh * np * AD + (int64_t)qt * 32 * AD;
  const T* DO = bf.dor + rh * np * AD + (int64_t)qt * 32 * AD;
  const T* K = bf.kr + rh * np * AD;
  const T* KT = bf.kt + rh * AD * np;
  const T* V = bf.vr + rh * np * AD;
  const T* Bh = bf.bias + ((int64_t)b * H + h) * N * N;
  const float* km = bf.kmask + br * np;
  const float mq = bf.mrow[rh * np + q];
  const float lq = bf.linv[rh * np + q];
  const float dq_ = bf.dd[rh * np + q];

  f32x16 dq = zero16();
  for (int kt = 0; kt < tiles1; ++kt) {
    const f32x16 sa = qk_tile<T>(K + (int64_t)kt * 32 * AD, Q);   // [key][q]: lane = q
    const f32x16 pa = qk_tile<T>(V + (int64_t)kt * 32 * AD, DO);  // dP^T
    float ds[16];
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const int k0 = kt * 32 + 8 * g + 4 * half;
      const f32x4 k4 = *reinterpret_cast<const f32x4*>(km + k0);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int key = k0 + e;
        const float bv = (q < N && key < N) ? to_f32(Bh[(int64_t)q * N + key]) : 0.f;
        const float s = score_of(sa[4 * g + e], scale, bv, k4[e], key < N);
        const float pr = __expf(s - mq) * lq;
        ds[4 * g + e] = pr * (pa[4 * g + e] - dq_);
      }
    }
    Frag<T> fs[2], fk[2];
    vals_to_frags<T>(fs, ds);
    dmajor_frags<T>(fk, KT, np, kt * 32);
    mma(dq, fk[0], fs[0]);
    mma(dq, fk[1], fs[1]);
  }
  T* dqo = bf.dq + (rh * np + q) * AD;
#pragma unroll
  for (int g = 0; g < 4; ++g)
    store4(dqo + 8 * g + 4 * half, scale * dq[4 * g], scale * dq[4 * g + 1], scale * dq[4 * g + 2],
           scale * dq[4 * g + 3]);
}

// ---------------------------------------------------------------------------
// dbias: per (batch, head, 32 queries, 32 keys), summed over the rows; lane = query
// ---------------------------------------------------------------------------
template <typename T, int H>
__global__ __launch_bounds__(256) void attn_bwd_dbias_kernel(AttnBwdBufs<T> bf, int B, int N, int np,
                                                             float scale) {
  const int lane = threadIdx.x & 63, half = lane >> 5, t32 = lane & 31;
  const int t1 = np / 32;
  const int64_t tile = (int64_t)blockIdx.x * 4 + wave_id();
  if (tile >= (int64_t)B * H * t1 * t1) return;
  const int kt = (int)(tile % t1);
  const int qt = (int)((tile / t1) % t1);
  const int h = (int)((tile / ((int64_t)t1 * t1)) % H);
  const int b = (int)(tile / ((int64_t)t1 * t1 * H));
  const int q = qt * 32 + t32;
  const T* Bh = bf.bias + ((int64_t)b * H + h) * N * N;
  float bv[16];
#pragma unroll
  for (int g = 0; g < 4; ++g)
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int key = kt * 32 + 8 * g + 4 * half + e;
      bv[4 * g + e] = (q < N && key < N) ? to_f32(Bh[(int64_t)q * N + key]) : 0.f;
    }
  float acc[16];
#pragma unroll
  for (int e = 0; e < 16; ++e) acc[e] = 0.f;
  for (int r = 0; r < N; ++r) {
    const int64_t br = (int64_t)b * N + r;
    const int64_t rh = br * H + h;
    const f32x16 sa = qk_tile<T>(bf.kr + (rh * np + (int64_t)kt * 32) * AD,
                                 bf.qr + (rh * np + (int64_t)qt * 32) * AD);
    const f32x16 pa = qk_tile<T>(bf.vr + (rh * np + (int64_t)kt * 32) * AD,
                                 bf.dor + (rh * np + (int64_t)qt * 32) * AD);
    const float mq = bf.mrow[rh * np + q];
    const float lq = bf.linv[rh * np + q];
    const float dq_ = bf.dd[rh * np + q];
    const float* km = bf.kmask + br * np;
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const int k0 = kt * 32 + 8 * g + 4 * half;
      const f32x4 k4 = *reinterpret_cast<const f32x4*>(km + k0);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float s = score_of(sa[4 * g + e], scale, bv[4 * g + e], k4[e], k0 + e < N);
        const float pr = __expf(s - mq) * lq;
        acc[4 * g + e] += pr * (pa[4 * g + e] - dq_);
      }
    }
  }
  if (q >= N) return;
  float* dst = bf.db + (((int64_t)b * H + h) * N + q) * N;
#pragma unroll
  for (int g = 0; g < 4; ++g)
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int key = kt * 32 + 8 * g + 4 * half + e;
      if (key < N) dst[key] = acc[4 * g + e];
    }
}

// ---------------------------------------------------------------------------
// (row, head) kernels of the bf16 path (np <= 1024): one 8-wave block per
// (row, head).  The operands every wave of the block reads (Q and dO for
// dK / dV, K and V for dQ) sit in LDS as [np][32] bf16 rows of 64 bytes, with
// 16-byte chunk c of row p at chunk c ^ ((p >> 2) & 3).  They are read both
// as fragments with d along k (ds_read_b128, conflict free) and transposed,
// with positions along k in the accumulator order of vals_to_frags
// (ds_read_b64_tr_b16).  Scores are taken in log2 units: with acc = bias /
// scale + q.k (the MFMA accumulates onto the fragment-order bias copies),
// s * log2(e) - lse2 = fma(acc, scale * log2(e), -lse2) and P = 2^that, where
// lse2 = (m + log l) * log2(e) of the query.  A row without a valid key
// attends uniformly (P = 1/l = 1/N over its real keys), as in
// attn_bwd_fwd_kernel.
// ---------------------------------------------------------------------------
constexpr int kRhWaves = 8;


// [np][32] rows of two operands of one (row, head) into swizzled LDS rows:
// np / 16 copies of 1 KiB each, spread over the block's waves.  The caller
// waits for its copies and synchronises the block.
__device__ __forceinline__ void rows2_to_lds(const bf16* a, char* la, const bf16* b, char* lb, int np) {
  const int lane = threadIdx.x & 63;
  const int wave = wave_id();
  const uint32_t rin = (uint32_t)lane >> 2;  // row within the copy (16 rows of 64 bytes)
  const uint32_t voff = rin * 64 + ((((uint32_t)lane & 3) ^ ((rin >> 2) & 3)) << 4);
  const int per = np / 16;
  for (int c = wave; c < 2 * per; c += kRhWaves) {
    const bool second = c >= per;
    const int cc = second ? c - per : c;
    g2lds16_sv(reinterpret_cast<const char*>(second ? b : a) + cc * 1024, voff,
               lds_addr(second ? lb : la) + cc * 1024);
  }
}

// Per-lane byte offsets into a swizzled 32-row tile.
struct RhOffsets {
  int nrm[2];  // fragment with rows = positions (lane&31), k = d 16m .. 16m+15 (k-step m)
  int tr[2];   // transposed reads: rows = d, k = positions 4(lane>>5) + {0..3, 8..11} (+ 1024 for the
               // positions 16..31 of the tile)
  __device__ __forceinline__ RhOffsets() {
    const int lane = threadIdx.x & 63;
    const int half = lane >> 5, t32 = lane & 31;
    const int sw = (t32 >> 2) & 3;
#pragma unroll
    for (int m = 0; m < 2; ++m) nrm[m] = t32 * 64 + (((2 * m + half) ^ sw) << 4);
    // ds_read_b64_tr_b16: within 16 lanes, lane L takes element L%4 of the 4
    // elements at the addresses of lanes L/4, 4 + L/4, 8 + L/4, 12 + L/4.
    // Lane j of group G supplies row 4(G>>1) + j/4 (+8), columns
    // 16(G&1) + 4(j&3) .. +3.
    const int G = lane >> 4, j = lane & 15;
    const int chunk = 2 * (G & 1) + ((j & 3) >> 1);
#pragma unroll
    for (int p = 0; p < 2; ++p)
      tr[p] = (4 * (G >> 1) + (j >> 2) + 8 * p) * 64 + ((chunk ^ ((G >> 1) + 2 * p)) << 4) + 8 * (j & 1);
  }
};

__device__ __forceinline__ Frag<bf16> lds_frag(const char* p) {
  Frag<bf16> f;
  f.load(reinterpret_cast<const bf16*>(p));
  return f;
}

// Transposed fragment gp (positions 16gp .. 16gp+15 of the tile at `tile`).
__device__ __forceinline__ Frag<bf16> lds_frag_tr(const char* tile, const RhOffsets& o, int gp) {
  typedef short s16x8 __attribute__((ext_vector_type(8)));
  const s16x4 p0 = lds_read_tr16(tile + gp * 1024 + o.tr[0]);
  const s16x4 p1 = lds_read_tr16(tile + gp * 1024 + o.tr[1]);
  const s16x8 v8 = {p0[0], p0[1], p0[2], p0[3], p1[0], p1[1], p1[2], p1[3]};
  Frag<bf16> f;
  f.v = __builtin_bit_cast(bf16x8, v8);
  return f;
}

// Does row br have a valid key?  (wave-uniform)
__device__ __forceinline__ bool rh_row_valid(const float* km_row, int N) {
  const int lane = threadIdx.x & 63;
  bool any = false;
  for (int k0 = 0; k0 < N; k0 += 64) {
    const int k = k0 + lane;
    any = any || (k < N && km_row[k] > 0.5f);
  }
  return __ballot(any) != 0ull;
}

// lse2 of query q of (row, head) rh: (m + log l) log2(e), or -log2(1/l) when
// the row has no valid key (its scores are then taken as 0)
__device__ __forceinline__ float rh_lse2(const AttnBwdBufs<bf16>& bf, int64_t idx, bool row_valid) {
  const float li = bf.linv[idx];
  return row_valid ? (bf.mrow[idx] - logf(li)) * kLog2e : -log2f(li);
}

// l in [2^-60, 2^64], tested on the bits: positive floats order as unsigned
// integers; NaN, zero, negative values and infinity fall outside.
__device__ __forceinline__ bool l_in_range_bits(float l) {
  return __float_as_uint(l) - 0x21800000u <= 0x5F800000u - 0x21800000u;
}

// One fp32 bias tile in fragment order (lane * 4 already in `p`): 4 loads of
// 16 bytes a lane, and the accumulator they initialise.
__device__ __forceinline__ void load_bias_tile(f32x4* dst, const float* p) {
#pragma unroll
  for (int g = 0; g < 4; ++g) dst[g] = *reinterpret_cast<const f32x4*>(p + g * 256);
}
__device__ __forceinline__ f32x16 bias_acc(const f32x4* v) {
  f32x16 a;
#pragma unroll
  for (int g = 0; g < 4; ++g)
#pragma unroll
    for (int rr = 0; rr < 4; ++rr) a[4 * g + rr] = v[g][rr];
  return a;
}

// Forward recompute: block (row, head), wave w owns query tiles w, w + 8, ...;
// lane = query.  A pass without a running maximum (m = 0, as in the forward
// flash kernel), and where its l leaves the safe range an online softmax over
// the key tiles with the exact running maximum; writes O (normalised), m
// (natural units) and 1/l like attn_bwd_fwd_kernel.  Padded queries attend uniformly, so that their O,
// m and l stay finite.
template <int NPM>
__global__ __launch_bounds__(64 * kRhWaves) void attn_bwd_fwd_rh_kernel(AttnBwdBufs<bf16> bf, int B,
                                                                     int N, int np, float scale,
                                                                     int exact_only) {
  constexpr int H = 4;
  __shared__ __attribute__((aligned(1024))) char ks[NPM * 64];
  __shared__ __attribute__((aligned(1024))) char vs[NPM * 64];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int half = lane >> 5, t32 = lane & 31;
  const int nt = np / 32;
  const int64_t rows = (int64_t)B * N;
  const int64_t lin = xcd_remap(blockIdx.x, gridDim.x);
  const int h = (int)(lin / rows);
  const int64_t br = lin - (int64_t)h * rows;
  const int b = (int)(br / N);
  const int64_t rh = br * H + h;
  rows2_to_lds(bf.kr + rh * np * AD, ks, bf.vr + rh * np * AD, vs, np);
  const float* km_row = bf.kmask + br * np;
  const bool row_valid = rh_row_valid(km_row, N);
  uint32_t kxv = 0;
  for (int k0 = 0; k0 < np; k0 += 64) {
    const int k = k0 + lane;
    const bool ex = k < np ? (row_valid ? !(km_row[k] > 0.5f) : k >= N) : true;
    const unsigned long long eb = __ballot(ex);
    const int w0 = k0 >> 5;
    if (lane == w0) kxv = (uint32_t)eb;
    if (lane == w0 + 1) kxv = (uint32_t)(eb >> 32);
  }
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();

  const RhOffsets off;
  const float c2 = scale * kLog2e;
  const int nk = (N + 31) / 32;
  const float* bT = bf.biasT + ((int64_t)b * H + h) * np * np + lane * 4;
  for (int qt = wave; qt < nt; qt += kRhWaves) {
    const int q = qt * 32 + t32;
    const bf16* qrow = bf.qr + (rh * np + q) * AD + 8 * half;
    Frag<bf16> qf[2];
#pragma unroll
    for (int m = 0; m < 2; ++m) qf[m].load(qrow + 16 * m);
    // scores taken as 0 (uniform attention): rows without a valid key, padded
    // queries (their scores are finite, so a zero factor gives 0)
    const float c2l = (!row_valid || q >= N) ? 0.f : c2;
    const float* btile = bT + (int64_t)qt * nt * 1024;
    // scores of key tile kt in log2 units (bias tile in bias), excluded keys at -inf
    auto scores = [&](int kt, float* s2, const f32x4* bias) {
      f32x16 sc = bias_acc(bias);
      if (row_valid) {
#pragma unroll
        for (int m = 0; m < 2; ++m) mma(sc, lds_frag(ks + kt * 2048 + off.nrm[m]), qf[m]);  // S^T: rows key, cols q
      } else {
        sc = zero16();
      }
#pragma unroll
      for (int e = 0; e < 16; ++e) s2[e] = sc[e] * c2l;
      const unsigned kx = __builtin_amdgcn_readlane(kxv, kt);
      if (kx != 0u) {
        const unsigned kl = kx >> (4 * half);
#pragma unroll
        for (int g = 0; g < 4; ++g)
#pragma unroll
          for (int rr = 0; rr < 4; ++rr)
            if (__builtin_amdgcn_ubfe(kl, 8 * g + rr, 1)) s2[4 * g + rr] = -INFINITY;
      }
    };
    // Fast pass: P = 2^s with no running maximum (m = 0), exact while every
    // 2^s stays in range, which l shows: l in [2^-60, 2^64] (the forward
    // flash kernel's test).  Otherwise (or with exact_only, for tests) the
    // exact pass below redoes the tile.  Bias tiles in two alternating
    // register sets, loaded one key tile ahead.
    float m2 = 0.f, l = 0.f;
    f32x16 o = zero16();
    auto fast_unit = [&](int kt, const f32x4* cur, f32x4* nxt) {
      load_bias_tile(nxt, btile + (kt + 1 < nk ? kt + 1 : kt) * 1024);
      float s2[16], pv[16], ps = 0.f;
      scores(kt, s2, cur);
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        pv[e] = __builtin_amdgcn_exp2f(s2[e]);
        ps += pv[e];
      }
      l += ps;
      Frag<bf16> fp[2];
      vals_to_frags<bf16>(fp, pv);
#pragma unroll
      for (int gp = 0; gp < 2; ++gp) mma(o, lds_frag_tr(vs + kt * 2048, off, gp), fp[gp]);  // O^T += V^T P^T
    };
    if (!exact_only) {
      f32x4 ba[4], bb[4];
      load_bias_tile(ba, btile);
      for (int kt = 0; kt < nk; kt += 2) {
        fast_unit(kt, ba, bb);
        if (kt + 1 < nk) fast_unit(kt + 1, bb, ba);
      }
    }
    l += __shfl_xor(l, 32);
    if (exact_only || __ballot(!l_in_range_bits(l)) != 0ull) {
      m2 = -INFINITY;
      l = 0.f;
      o = zero16();
      for (int kt = 0; kt < nk; ++kt) {
        float s2[16];
        {
          f32x4 bt[4];
          load_bias_tile(bt, btile + kt * 1024);
          scores(kt, s2, bt);
        }
        float mt = s2[0];
#pragma unroll
        for (int e = 1; e < 16; ++e) mt = fmaxf(mt, s2[e]);
        mt = fmaxf(mt, __shfl_xor(mt, 32));
        const float mn = fmaxf(m2, mt);
        const bool none = mn == -INFINITY;  // no key so far
        const float alpha = none ? 1.f : __builtin_amdgcn_exp2f(m2 - mn);
        float pv[16], ps = 0.f;
#pragma unroll
        for (int e = 0; e < 16; ++e) {
          pv[e] = none ? 0.f : __builtin_amdgcn_exp2f(s2[e] - mn);
          ps += pv[e];
        }
        l = l * alpha + ps;
        m2 = mn;
#pragma unroll
        for (int e = 0; e < 16; ++e) o[e] *= alpha;
        Frag<bf16> fp[2];
        vals_to_frags<bf16>(fp, pv);
#pragma unroll
        for (int gp = 0; gp < 2; ++gp) mma(o, lds_frag_tr(vs + kt * 2048, off, gp), fp[gp]);  // O^T += V^T P^T
      }
      l += __shfl_xor(l, 32);
    }
    const float li = 1.0f / l;
    {
      float ov[16];
#pragma unroll
      for (int e = 0; e < 16; ++e) ov[e] = o[e] * li;
      store_row32_bf16(bf.o + (rh * np + q) * AD, ov);
    }
    if (half == 0) {
      bf.mrow[rh * np + q] = row_valid ? (q < N ? m2 * (1.0f / kLog2e) : 0.f) : kMaskScore;
      bf.linv[rh * np + q] = li;
    }
  }
}

// dK and dV: block (row, head), wave w owns key tiles w, w + 8, ...; lane = key.
// Padded queries carry lse2 = +inf (P = 0) and D = 0; an excluded key's
// column of dK^T and dV^T (its lane) is zeroed at the end instead of its P
// values per tile: each column of an MFMA product reads only that column of
// the B operand.  The bias tiles alternate between two register sets, so the
// next tile's loads go out before the current one is used, without copies.
template <int NPM>
__global__ __launch_bounds__(64 * kRhWaves) void attn_bwd_dkdv_rh_kernel(AttnBwdBufs<bf16> bf, int B,
                                                                      int N, int np, float scale) {
  constexpr int H = 4;
  // lse2 and D first, so that their offsets fit the LDS instructions' 16-bit
  // immediate; then Q and dO rows
  __shared__ __attribute__((aligned(1024))) char lds[8 * NPM + 2 * NPM * 64];
  float* const lse_s = reinterpret_cast<float*>(lds);
  float* const dd_s = lse_s + NPM;
  char* const qs = lds + 8 * NPM;
  char* const dos = qs + NPM * 64;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int half = lane >> 5, t32 = lane & 31;
  const int nt = np / 32;
  const int64_t rows = (int64_t)B * N;
  const int64_t lin = xcd_remap(blockIdx.x, gridDim.x);
  const int h = (int)(lin / rows);  // head-major: the blocks of one XCD share one head's bias
  const int64_t br = lin - (int64_t)h * rows;
  const int b = (int)(br / N);
  const int64_t rh = br * H + h;
  rows2_to_lds(bf.qr + rh * np * AD, qs, bf.dor + rh * np * AD, dos, np);
  const float* km_row = bf.kmask + br * np;
  const bool row_valid = rh_row_valid(km_row, N);
  for (int q = tid; q < np; q += 64 * kRhWaves) {
    lse_s[q] = q < N ? rh_lse2(bf, rh * np + q, row_valid) : INFINITY;
    dd_s[q] = q < N ? bf.dd[rh * np + q] : 0.f;
  }
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();

  const RhOffsets off;
  const float c2 = scale * kLog2e;
  const int nq = (N + 31) / 32;  // query tiles with a real query
  const float* bS = bf.biasS + ((int64_t)b * H + h) * np * np + lane * 4;
  for (int kt = wave; kt < nt; kt += kRhWaves) {
    const int key = kt * 32 + t32;
    const bf16* krow = bf.kr + (rh * np + key) * AD + 8 * half;
    const bf16* vrow = bf.vr + (rh * np + key) * AD + 8 * half;
    Frag<bf16> kf[2], vf[2];
#pragma unroll
    for (int m = 0; m < 2; ++m) {
      kf[m].load(krow + 16 * m);
      vf[m].load(vrow + 16 * m);
    }
    // excluded key (no weight): padding, or masked in a row with a valid key
    const bool excl = row_valid ? !(km_row[key] > 0.5f) : key >= N;
    const float* btile = bS + (int64_t)kt * nt * 1024;
    f32x16 dk = zero16(), dv = zero16();
    // query tile qt with its bias in cur; the next tile's bias goes to nxt
    auto unit = [&](int qt, const f32x4* cur, f32x4* nxt) {
      load_bias_tile(nxt, btile + (qt + 1 < nq ? qt + 1 : qt) * 1024);
      const char* qtile = qs + qt * 2048;
      const char* dtile = dos + qt * 2048;
      f32x16 sc = bias_acc(cur);
      if (row_valid) {
#pragma unroll
        for (int m = 0; m < 2; ++m) mma(sc, lds_frag(qtile + off.nrm[m]), kf[m]);  // S: rows q, cols key
      } else {
        sc = zero16();
      }
      f32x16 dp = mma0(lds_frag(dtile + off.nrm[0]), vf[0]);
      mma(dp, lds_frag(dtile + off.nrm[1]), vf[1]);
      float pv[16], dsv[16];
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int q0 = qt * 32 + 8 * g + 4 * half;
        const f32x4 l4 = *reinterpret_cast<const f32x4*>(lse_s + q0);
        const f32x4 d4 = *reinterpret_cast<const f32x4*>(dd_s + q0);
#pragma unroll
        for (int rr = 0; rr < 4; ++rr) {
          pv[4 * g + rr] = __builtin_amdgcn_exp2f(fmaf(sc[4 * g + rr], c2, -l4[rr]));
          dsv[4 * g + rr] = pv[4 * g + rr] * (dp[4 * g + rr] - d4[rr]);
        }
      }
      Frag<bf16> fp[2], fs[2];
      vals_to_frags<bf16>(fp, pv);
      vals_to_frags<bf16>(fs, dsv);
#pragma unroll
      for (int gp = 0; gp < 2; ++gp) {
        mma(dv, lds_frag_tr(dtile, off, gp), fp[gp]);  // dV^T[d][key] += dO^T P
        mma(dk, lds_frag_tr(qtile, off, gp), fs[gp]);  // dK^T[d][key] += Q^T dS
      }
    };
    f32x4 ba[4], bb[4];
    load_bias_tile(ba, btile);
    for (int qt = 0; qt < nq; qt += 2) {
      unit(qt, ba, bb);
      if (qt + 1 < nq) unit(qt + 1, bb, ba);
    }
    if (excl) {
      dk = zero16();
      dv = zero16();
    }
    {
      float kv[16], vv[16];
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        kv[e] = scale * dk[e];
        vv[e] = dv[e];
      }
      store_row32_bf16(bf.dk + (rh * np + key) * AD, kv);
      store_row32_bf16(bf.dv + (rh * np + key) * AD, vv);
    }
  }
}

// dQ: block (row, head), wave w owns query tiles w, w + 8, ...; lane = query.
// Bias tiles in two alternating register sets, as in the dK / dV kernel.
template <int NPM>
__global__ __launch_bounds__(64 * kRhWaves) __attribute__((amdgpu_waves_per_eu(4))) void attn_bwd_dq_rh_kernel(AttnBwdBufs<bf16> bf, int B,
                                                                    int N, int np, float scale) {
  constexpr int H = 4;
  __shared__ __attribute__((aligned(1024))) char ks[NPM * 64];
  __shared__ __attribute__((aligned(1024))) char vs[NPM * 64];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int half = lane >> 5, t32 = lane & 31;
  const int nt = np / 32;
  const int64_t rows = (int64_t)B * N;
  const int64_t lin = xcd_remap(blockIdx.x, gridDim.x);
  const int h = (int)(lin / rows);
  const int64_t br = lin - (int64_t)h * rows;
  const int b = (int)(br / N);
  const int64_t rh = br * H + h;
  rows2_to_lds(bf.kr + rh * np * AD, ks, bf.vr + rh * np * AD, vs, np);
  const float* km_row = bf.kmask + br * np;
  const bool row_valid = rh_row_valid(km_row, N);
  // excluded keys (padding, and masked keys of a row with a valid key): bit j
  // of lane t's word is key 32t + j
  uint32_t kxv = 0;
  for (int k0 = 0; k0 < np; k0 += 64) {
    const int k = k0 + lane;
    const bool ex = k < np ? (row_valid ? !(km_row[k] > 0.5f) : k >= N) : true;
    const unsigned long long eb = __ballot(ex);
    const int w0 = k0 >> 5;
    if (lane == w0) kxv = (uint32_t)eb;
    if (lane == w0 + 1) kxv = (uint32_t)(eb >> 32);
  }
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();

  const RhOffsets off;
  const float c2 = scale * kLog2e;
  const int nk = (N + 31) / 32;  // key tiles with a real key
  const float* bT = bf.biasT + ((int64_t)b * H + h) * np * np + lane * 4;
  for (int qt = wave; qt < nt; qt += kRhWaves) {
    const int q = qt * 32 + t32;
    const bf16* qrow = bf.qr + (rh * np + q) * AD + 8 * half;
    const bf16* drow = bf.dor + (rh * np + q) * AD + 8 * half;
    Frag<bf16> qf[2], df[2];
#pragma unroll
    for (int m = 0; m < 2; ++m) {
      qf[m].load(qrow + 16 * m);
      df[m].load(drow + 16 * m);
    }
    const float lse2 = rh_lse2(bf, rh * np + q, row_valid);
    const float dq_ = bf.dd[rh * np + q];
    const bool qpad = q >= N;  // a padded query's column of dQ^T is zeroed at the end
    const float* btile = bT + (int64_t)qt * nt * 1024;
    f32x16 dq = zero16();
    // key tile kt with its bias in cur; the next tile's bias goes to nxt
    auto unit = [&](int kt, const f32x4* cur, f32x4* nxt) {
      load_bias_tile(nxt, btile + (kt + 1 < nk ? kt + 1 : kt) * 1024);
      const char* ktile = ks + kt * 2048;
      const char* vtile = vs + kt * 2048;
      f32x16 sc = bias_acc(cur);
      if (row_valid) {
#pragma unroll
        for (int m = 0; m < 2; ++m) mma(sc, lds_frag(ktile + off.nrm[m]), qf[m]);  // S^T: rows key, cols q
      } else {
        sc = zero16();
      }
      f32x16 dp = mma0(lds_frag(vtile + off.nrm[0]), df[0]);  // dP^T
      mma(dp, lds_frag(vtile + off.nrm[1]), df[1]);
      float pv[16];
#pragma unroll
      for (int e = 0; e < 16; ++e) pv[e] = __builtin_amdgcn_exp2f(fmaf(sc[e], c2, -lse2));
      const unsigned kx = __builtin_amdgcn_readlane(kxv, kt);
      if (kx != 0u) {
        // this lane's keys 8g + 4*half + rr: bits 8g + rr after the shift
        const unsigned kl = kx >> (4 * half);
#pragma unroll
        for (int g = 0; g < 4; ++g)
#pragma unroll
          for (int rr = 0; rr < 4; ++rr)
            if (__builtin_amdgcn_ubfe(kl, 8 * g + rr, 1)) pv[4 * g + rr] = 0.f;
      }
      float dsv[16];
#pragma unroll
      for (int e = 0; e < 16; ++e) dsv[e] = pv[e] * (dp[e] - dq_);
      Frag<bf16> fs[2];
      vals_to_frags<bf16>(fs, dsv);
#pragma unroll
      for (int gp = 0; gp < 2; ++gp) mma(dq, lds_frag_tr(ktile, off, gp), fs[gp]);  // dQ^T[d][q] += K^T dS^T
    };
    f32x4 ba[4], bb[4];
    load_bias_tile(ba, btile);
    for (int kt = 0; kt < nk; kt += 2) {
      unit(kt, ba, bb);
      if (kt + 1 < nk) unit(kt + 1, bb, ba);
    }
    if (qpad) dq = zero16();
    {
      float qv[16];
#pragma unroll
      for (int e = 0; e < 16; ++e) qv[e] = scale * dq[e];
      store_row32_bf16(bf.dq + (rh * np + q) * AD, qv);
    }
  }
}

// dB of the bf16 path (np <= 512): block (batch b, head h, pair of query
// tiles, chunk of rows).  The block's waves walk the chunk's rows together,
// each owning key tiles w and w + 8 (lane = query, S^T orientation as in dQ)
// for both query tiles, so each K and V fragment read serves two tiles.  For
// every row, K and V of the row and the two query tiles of Q and dO come into
// LDS (double buffered: the copies of row r + 1 go out before row r is
// computed), and each wave adds dS of its tiles into fp32 accumulators.  The
// chunk's sums go to a partial buffer in fragment order (the biasT layout),
// summed over the chunks by attn_bwd_dbias_reduce_kernel.  Blocks of one
// (b, chunk, head) are consecutive, so the blocks that read the same K and V
// rows share an XCD's L2.  Two query tiles a block halve the K/V bytes moved
// per unit of work and make the launch one round of blocks at N = 512.
constexpr int kDbChunks = 8;  // row chunks per batch element (at most)
constexpr int kDbQt = 2;      // query tiles per block

template <int NPM>
__global__ __launch_bounds__(64 * kRhWaves) void attn_bwd_dbias_rh_kernel(AttnBwdBufs<bf16> bf,
                                                                       float* __restrict__ part, int B,
                                                                       int N, int np, int nch, int rpc,
                                                                       float scale) {
  constexpr int H = 4;
  constexpr int QP = kDbQt;
  static_assert(NPM <= 512, "two key tiles per wave");
  constexpr int BUF = 2 * NPM * 64 + QP * 4096;  // K rows, V rows, then Q and dO tiles of each query tile
  // per-row scalars: m, 1/l and D of the block's 64 queries (768 bytes,
  // loaded by wave 0), then the mask values of each wave's key tiles (256
  // bytes a wave)
  constexpr int SCB = 768 + kRhWaves * 256;
  __shared__ __attribute__((aligned(1024))) char lds[2 * BUF];
  __shared__ __attribute__((aligned(256))) char pf_scratch[kRhWaves][256];  // L2 prefetch landing area
  __shared__ __attribute__((aligned(256))) char row_sc[2 * SCB];             // per-row scalars, two rows
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int half = lane >> 5, t32 = lane & 31;
  const int nt = np / 32;
  const int nq = (N + 31) / 32;
  const int nqp = (nq + QP - 1) / QP;
  const int64_t lin = xcd_remap(blockIdx.x, gridDim.x);
  const int qp = (int)(lin % nqp);
  int64_t rest = lin / nqp;
  const int h = (int)(rest % H);
  rest /= H;
  const int c = (int)(rest % nch);
  const int b = (int)(rest / nch);
  const int r0 = c * rpc;
  const int r1 = min(N, r0 + rpc);
  const int qt0 = qp * QP;
  const bool two = qt0 + 1 < nq;  // block-uniform: a second query tile exists
  int qtq[QP];                    // query tile q (the second reads the first's data when absent)
  qtq[0] = qt0;
  qtq[1] = two ? qt0 + 1 : qt0;
  const int kv_bytes = np * 64;
  const int ncopy = np / 8 + 4 * QP;  // 1 KiB copies per row: K, V, and a Q and dO tile per query tile

  // copies of row r into buffer u
  const uint32_t rin = (uint32_t)lane >> 2;
  const uint32_t voff = rin * 64 + ((((uint32_t)lane & 3) ^ ((rin >> 2) & 3)) << 4);
  auto issue_row = [&](int r, int u) {
    const int64_t rh = ((int64_t)b * N + r) * H + h;
    const char* kb = reinterpret_cast<const char*>(bf.kr + rh * np * AD);
    const char* vb = reinterpret_cast<const char*>(bf.vr + rh * np * AD);
    const char* qb0 = reinterpret_cast<const char*>(bf.qr + (rh * np + qtq[0] * 32) * AD);
    const char* db0 = reinterpret_cast<const char*>(bf.dor + (rh * np + qtq[0] * 32) * AD);
    const char* qb1 = reinterpret_cast<const char*>(bf.qr + (rh * np + qtq[1] * 32) * AD);
    const char* db1 = reinterpret_cast<const char*>(bf.dor + (rh * np + qtq[1] * 32) * AD);
    const uint32_t base = lds_addr(lds) + u * BUF;
    for (int i = wave; i < ncopy; i += kRhWaves) {
      const char* src;
      const int j = i - np / 8;  // copy j of the query tiles' 8
      if (i < np / 16) src = kb + i * 1024;
      else if (i < np / 8) src = vb + (i - np / 16) * 1024;
      else if (j < 2) src = qb0 + j * 1024;
      else if (j < 4) src = db0 + (j - 2) * 1024;
      else if (j < 6) src = qb1 + (j - 4) * 1024;
      else src = db1 + (j - 6) * 1024;
      // wave-uniform, but selected per copy: back into scalar registers
      // (readfirstlane returns int: widen each half as unsigned)
      const uint64_t sa = (uint64_t)(uintptr_t)src;
      const uint64_t su = ((uint64_t)(uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)(sa >> 32)) << 32) |
                          (uint64_t)(uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)sa);
      g2lds16_sv(reinterpret_cast<const char*>(su), voff, __builtin_amdgcn_readfirstlane(base + i * 1024));
    }
  };
  // Per-row scalars come into LDS like the rows, one row ahead, as 4-byte
  // direct loads: wave 0 brings m, 1/l and D of the 64 queries (lanes 0-31
  // the first tile's, 32-63 the second's), every wave the mask values of its
  // key tiles (lanes 0-31 tile w, 32-63 tile w + 8; a tile past the last
  // reads tile nt - 1, unused).
  const int kt0c = min(wave, nt - 1), kt1c = min(wave + kRhWaves, nt - 1);
  const int myq = qtq[half] * 32 + t32;  // the query this lane brings in
  auto issue_scalars = [&](int r, int u) {
    const int64_t br = (int64_t)b * N + r;
    const int64_t qi = (br * H + h) * np + myq;
    const uint32_t base = lds_addr(row_sc) + (uint32_t)(u * SCB);
    if (wave == 0) {
      g2lds4(bf.mrow + qi, base);
      g2lds4(bf.linv + qi, base + 256);
      g2lds4(bf.dd + qi, base + 512);
    }
    g2lds4(bf.kmask + br * np + (half ? kt1c : kt0c) * 32 + t32, base + 768 + wave * 256);
  };
  // L2 prefetch, two rows ahead: one 4-byte load a lane brings the row's K
  // and V lines (np / 2 lines of 128 bytes each; lane l of wave w takes line
  // 64w + l) into L2, so that the copies issued a row later hit there; it
  // lands in a per-wave LDS scratch area nothing reads.  Each row's top waits
  // for all but the newest load (this prefetch, issued after the row's
  // copies and scalars).
  const int gl = wave * 64 + lane;
  const uint32_t pf_lds = lds_addr(pf_scratch[wave]);
  auto prefetch_row = [&](int r) {
    const int64_t rh = ((int64_t)b * N + r) * H + h;
    const int kind = gl < np / 2 ? 0 : gl < np ? 1 : 2;
    const char* p = reinterpret_cast<const char*>((kind == 1 ? bf.vr : bf.kr) + rh * np * AD) +
                    (kind == 0 ? gl : kind == 1 ? gl - np / 2 : 0) * 128;
    g2lds4(p, pf_lds);
  };

  const RhOffsets off;
  const float c2 = scale * kLog2e;
  // bias tiles (h, qt, kt) of this wave's key tiles for both query tiles
  f32x16 bias[QP][2], acc[QP][2];
  const float* bT = bf.biasT + ((int64_t)b * H + h) * np * np + lane * 4;
#pragma unroll
  for (int q = 0; q < QP; ++q)
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int kt = min(wave + kRhWaves * i, nt - 1);
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const f32x4 v = *reinterpret_cast<const f32x4*>(bT + ((int64_t)qtq[q] * nt + kt) * 1024 + g * 256);
#pragma unroll
        for (int rr = 0; rr < 4; ++rr) bias[q][i][4 * g + rr] = v[rr];
      }
      acc[q][i] = zero16();
    }
  // Every load in the row loop is a direct-to-LDS copy issued from asm, so
  // the compiler adds no wait of its own there; the bias tiles (ordinary
  // loads) have landed before the loop.
  issue_scalars(r0, 0);
  issue_row(r0, 0);
  __builtin_amdgcn_s_waitcnt(vmcnt_imm<0>());
  for (int r = r0; r < r1; ++r) {
    const int u = (r - r0) & 1;
    // this wave's copies of row r landed (the prefetch of row r + 1, issued
    // after them, may still be in flight)
    __builtin_amdgcn_s_waitcnt(vmcnt_imm<1>());
    barrier_only();  // every wave's copies landed; row r - 1's buffer is free
    if (r + 1 < r1) {
      issue_scalars(r + 1, u ^ 1);
      issue_row(r + 1, u ^ 1);
    }
    prefetch_row(min(r + 2, r1 - 1));
    const char* buf = lds + u * BUF;
    const float* sq = reinterpret_cast<const float*>(row_sc + u * SCB);
    const float* skm = reinterpret_cast<const float*>(row_sc + u * SCB + 768 + wave * 256);
    // a row without a valid key stores m = -1e9 for every query
    const bool row_valid = __ballot(sq[t32] != kMaskScore) != 0ull;
    float lse2[QP], dd[QP];
    Frag<bf16> qf[QP][2], df[QP][2];
#pragma unroll
    for (int q = 0; q < QP; ++q) {
      // a padded query takes lse2 = +inf: P = 0
      const bool qpad = qtq[q] * 32 + t32 >= N;
      const float m = sq[32 * q + t32], li = sq[64 + 32 * q + t32];
      lse2[q] = qpad ? INFINITY : row_valid ? (m - logf(li)) * kLog2e : -log2f(li);
      dd[q] = qpad ? 0.f : sq[128 + 32 * q + t32];
      const char* qtile = buf + 2 * kv_bytes + q * 4096;
#pragma unroll
      for (int m2 = 0; m2 < 2; ++m2) {
        qf[q][m2] = lds_frag(qtile + off.nrm[m2]);
        df[q][m2] = lds_frag(qtile + 2048 + off.nrm[m2]);
      }
    }
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int kt = wave + kRhWaves * i;
      if (kt >= nt) break;
      const int key = kt * 32 + t32;
      const bool ex = row_valid ? !(skm[32 * i + t32] > 0.5f) : key >= N;
      const unsigned kx = (unsigned)__ballot(ex);  // lanes 0-31: the tile's 32 keys
      const char* ktile = buf + kt * 2048;
      const char* vtile = buf + kv_bytes + kt * 2048;
      const Frag<bf16> kf0 = lds_frag(ktile + off.nrm[0]), kf1 = lds_frag(ktile + off.nrm[1]);
      const Frag<bf16> vf0 = lds_frag(vtile + off.nrm[0]), vf1 = lds_frag(vtile + off.nrm[1]);
#pragma unroll
      for (int q = 0; q < QP; ++q) {
        if (q > 0 && !two) break;
        f32x16 sc = zero16();
        if (row_valid) {
          sc = bias[q][i];
          mma(sc, kf0, qf[q][0]);  // S^T: rows key, cols q
          mma(sc, kf1, qf[q][1]);
        }
        f32x16 dp = mma0(vf0, df[q][0]);  // dP^T
        mma(dp, vf1, df[q][1]);
        float pv[16];
#pragma unroll
        for (int e = 0; e < 16; ++e) pv[e] = __builtin_amdgcn_exp2f(fmaf(sc[e], c2, -lse2[q]));  // sc = 0 in an invalid row
        if (kx != 0u) {
          const unsigned kl = kx >> (4 * half);
#pragma unroll
          for (int g = 0; g < 4; ++g)
#pragma unroll
            for (int rr = 0; rr < 4; ++rr)
              if (__builtin_amdgcn_ubfe(kl, 8 * g + rr, 1)) pv[4 * g + rr] = 0.f;
        }
#pragma unroll
        for (int e = 0; e < 16; ++e) acc[q][i][e] += pv[e] * (dp[e] - dd[q]);
      }
    }
  }
  // the last prefetches land before the block's LDS can pass to another block
  __builtin_amdgcn_s_waitcnt(vmcnt_imm<0>());
  float* dst = part + ((int64_t)(b * nch + c) * H + h) * np * np + lane * 4;
#pragma unroll
  for (int q = 0; q < QP; ++q) {
    if (q > 0 && !two) break;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int kt = wave + kRhWaves * i;
      if (kt >= nt) break;
#pragma unroll
      for (int g = 0; g < 4; ++g)
        *reinterpret_cast<f32x4*>(dst + ((int64_t)qtq[q] * nt + kt) * 1024 + g * 256) =
            f32x4{acc[q][i][4 * g], acc[q][i][4 * g + 1], acc[q][i][4 * g + 2], acc[q][i][4 * g + 3]};
    }
  }
}

// db[b][h][q][k] = sum over the row chunks of the fragment-order partials.
// Thread t sums the t-th 16-byte piece of the fragment-order layout (keys
// 8g + 4 half .. +3 of query a in tile (h, qt, kt), as bias_frag_elem lays
// them out), so the partials are read in whole lines; a 256-thread block
// covers one 32 x 32 tile, whose 32 output rows of 128 bytes its four waves
// write together.  Tiles outside the N x N grid are skipped.
__global__ __launch_bounds__(256) void attn_bwd_dbias_reduce_kernel(const float* __restrict__ part,
                                                                    float* __restrict__ db, int B, int N,
                                                                    int np, int nch) {
  constexpr int H = 4;
  const int nt = np / 32;
  const int64_t tile = blockIdx.x;  // [B][H][qt][kt]
  const int kt = (int)(tile % nt), qt = (int)((tile / nt) % nt);
  const int64_t bh = tile / ((int64_t)nt * nt);
  if (qt * 32 >= N || kt * 32 >= N) return;  // block-uniform
  const int b = (int)(bh / H), h = (int)(bh % H);
  const int tid = threadIdx.x;
  const int g = tid >> 6, l = tid & 63;
  const int q = qt * 32 + (l & 31), k = kt * 32 + 8 * g + 4 * (l >> 5);
  const int64_t e = (((int64_t)h * nt + qt) * nt + kt) * 1024 + tid * 4;  // == bias_frag_elem(h, q, k, np)
  const int64_t slab = (int64_t)H * np * np;
  const float* src = part + (int64_t)b * nch * slab + e;
  f32x4 s = {0.f, 0.f, 0.f, 0.f};
  for (int c = 0; c < nch; ++c) {
    const f32x4 v = *reinterpret_cast<const f32x4*>(src + c * slab);
#pragma unroll
    for (int j = 0; j < 4; ++j) s[j] += v[j];
  }
  if (q >= N) return;
  float* dst = db + (((int64_t)b * H + h) * N + q) * N + k;
#pragma unroll
  for (int j = 0; j < 4; ++j)
    if (k + j < N) dst[j] = s[j];
}

// ---------------------------------------------------------------------------
// pro: dxn and the LayerNorm backward; per 32-position tile of one row
// ---------------------------------------------------------------------------
template <typename T, int C, int H>
__global__ __launch_bounds__(256) void attn_bwd_pro_kernel(const T* __restrict__ x, T* __restrict__ dx,
                                                           AttnBwdW<T> w, AttnBwdBufs<T> bf, int B,
                                                           int N, int np, int starting, float eps) {
  constexpr int CH = H * AD;
  const int lane = threadIdx.x & 63, half = lane >> 5, t32 = lane & 31;
  const int jtiles = np / 32;
  const int64_t tile = (int64_t)blockIdx.x * 4 + wave_id();
  if (tile >= (int64_t)B * N * jtiles) return;
  const int jt = (int)(tile % jtiles);
  const int r = (int)((tile / jtiles) % N);
  const int b = (int)(tile / ((int64_t)jtiles * N));
  const int j = jt * 32 + t32;
  const bool valid = j < N;
  const int64_t xp = valid ? ((int64_t)b * N + (starting ? r : j)) * N + (starting ? j : r) : 0;
  const int64_t p = ((int64_t)b * N + r) * N + j;
  const int64_t pitch = bf.pitch;
  // column-major operand tiles: whole-tile transposed stores where possible
  const int64_t p0 = ((int64_t)b * N + r) * N + jt * 32;
  const bool fast = std::is_same<T, bf16>::value && jt * 32 + 32 <= N && N % 4 == 0;
  const CmTile cmt;

  RowHalf<C> rhx;
  load_row_half<T, C>(rhx, x + xp * C, valid);
  const f32x2 st = row_stats<C>(rhx, eps);

  f32x16 dzn[C / 32];
#pragma unroll
  for (int nt = 0; nt < C / 32; ++nt) dzn[nt] = zero16();
  const T* src[3] = {bf.dq, bf.dk, bf.dv};
  const T* wts[4] = {w.wt_q, w.wt_k, w.wt_v, w.wt_g};
#pragma unroll 1
  for (int kind = 0; kind < 4; ++kind) {
#pragma unroll 1
    for (int h = 0; h < H; ++h) {
      // this (kind, head)'s weight fragments first: their loads overlap the operand loads
      Frag<T> wf[C / 32][2];
#pragma unroll
      for (int nt2 = 0; nt2 < C / 32; ++nt2)
#pragma unroll
        for (int gp = 0; gp < 2; ++gp) load_wfrag<T>(wf[nt2][gp], wts[kind], nt2, 2 * h + gp, CH / 16);
      float d[16];
      // the loads are unconditional (a padded lane reads position j of the
      // padded slab, or pair p0 of the column-major planes) and selected
      // afterwards, so they go out together instead of one branch each
      if (kind < 3) {
        const T* s = src[kind] + ((((int64_t)b * N + r) * H + h) * np + j) * AD;
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const f32x4 v4 = load4f(s + 8 * g + 4 * half);
#pragma unroll
          for (int e = 0; e < 4; ++e) d[4 * g + e] = valid ? v4[e] : 0.f;
        }
        if constexpr (std::is_same<T, bf16>::value) {
          cmt.store(bf.cm_stack, pitch, p0, kind * CH + h * AD, d, fast, valid);
        } else if (valid) {
#pragma unroll
          for (int g = 0; g < 4; ++g)
#pragma unroll
            for (int e = 0; e < 4; ++e)
              bf.cm_stack[(int64_t)(kind * CH + h * AD + 8 * g + 4 * half + e) * pitch + p] =
                  cvt<T>(d[4 * g + e]);
        }
      } else {
        const int64_t ps = valid ? p : p0;
#pragma unroll
        for (int g = 0; g < 4; ++g)
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const float v = to_f32(bf.cm_stack[(int64_t)(3 * CH + h * AD + 8 * g + 4 * half + e) * pitch + ps]);
            d[4 * g + e] = valid ? v : 0.f;
          }
      }
      Frag<T> f[2];
      vals_to_frags<T>(f, d);
#pragma unroll
      for (int nt2 = 0; nt2 < C / 32; ++nt2)
#pragma unroll
        for (int gp = 0; gp < 2; ++gp) mma(dzn[nt2], wf[nt2][gp], f[gp]);
    }
  }
  // triangle bias: dxn += sum_h dB[h][r][j] W_b[h][.]
  float dtri[H];
#pragma unroll
  for (int h = 0; h < H; ++h) {
    dtri[h] = valid ? bf.db[(((int64_t)b * H + h) * N + r) * N + j] : 0.f;
    if (valid && half == 0) bf.cm_dtri[(int64_t)h * pitch + p] = cvt<T>(dtri[h]);
  }
  float xh[C / 2];
  float s1 = 0.f, s2 = 0.f;
#pragma unroll
  for (int nt = 0; nt < C / 32; ++nt)
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const int c0 = nt * 32 + 8 * g + 4 * half;
      const f32x4 x4 = valid ? load4f(x + xp * C + c0) : f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        float t = dzn[nt][4 * g + e];
#pragma unroll
        for (int h = 0; h < H; ++h) t += dtri[h] * w.wb_raw[h * C + c0 + e];
        dzn[nt][4 * g + e] = t;
        const float xv = (x4[e] - st[0]) * st[1];
        xh[16 * nt + 4 * g + e] = xv;
        const float dxh = w.ln_w[c0 + e] * t;
        s1 += dxh;
        s2 += dxh * xv;
      }
    }
  s1 += xor32(s1);
  s2 += xor32(s2);
  const float m1 = s1 * (1.0f / C), m2 = s2 * (1.0f / C);
  if constexpr (std::is_same<T, bf16>::value) {
#pragma unroll
    for (int nt = 0; nt < C / 32; ++nt) {
      float vt[16];
#pragma unroll
      for (int e = 0; e < 16; ++e) vt[e] = dzn[nt][e];
      cmt.store(bf.cm_xh, pitch, p0, nt * 32, &xh[16 * nt], fast, valid);
      cmt.store(bf.cm_dxn, pitch, p0, nt * 32, vt, fast, valid);
    }
  }
  if (!valid) return;
#pragma unroll
  for (int nt = 0; nt < C / 32; ++nt)
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const int c0 = nt * 32 + 8 * g + 4 * half;
      float o[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float xv = xh[16 * nt + 4 * g + e];
        const float t = dzn[nt][4 * g + e];
        o[e] = st[1] * (w.ln_w[c0 + e] * t - m1 - xv * m2);
        if constexpr (!std::is_same<T, bf16>::value) {
          bf.cm_xh[(int64_t)(c0 + e) * pitch + p] = cvt<T>(xv);
          bf.cm_dxn[(int64_t)(c0 + e) * pitch + p] = cvt<T>(t);
        }
      }
      store4(dx + xp * C + c0, o[0], o[1], o[2], o[3]);
    }
}

// ---------------------------------------------------------------------------
// pro, bf16: the same algebra as attn_bwd_pro_kernel in persistent blocks of
// 8 waves.  The kernel above reads the (kind, head) weight fragments of its
// 16 d W products from L2 (128 KiB a 32-position tile at c_in = 128) and
// holds them in registers (one wave a SIMD); here W^T of q, k, v and the gate
// (4 x c_in x c_h bf16), W_b and the LayerNorm weight sit in LDS, two waves a
// SIMD.  Whole tiles (32 valid positions, rows 16-byte aligned: N % 8 == 0)
// move their channel-major blocks through a per-wave LDS tile, 16 bytes a
// lane (the gate's d rows are read the same way); other tiles take the
// element path.  The rows of x are read again for the LayerNorm backward
// rather than kept (64 values a lane).
// ---------------------------------------------------------------------------
template <int C, int H>
__global__ __launch_bounds__(512) void attn_bwd_pro_lds_kernel(const bf16* __restrict__ x, bf16* __restrict__ dx,
                                                               AttnBwdW<bf16> w, AttnBwdBufs<bf16> bf, int B, int N,
                                                               int np, int starting, float eps, int64_t ntiles) {
  constexpr int CH = H * AD;
  constexpr int PW = C * CH;  // elements of one packed W^T
  __shared__ __attribute__((aligned(1024))) bf16 wl[4][PW];
  __shared__ __attribute__((aligned(16))) bf16 cst[8][kCmTile];
  __shared__ __attribute__((aligned(16))) float wbl[H * C];
  __shared__ __attribute__((aligned(16))) float lnw[C];
  copy_to_lds_async(wl[0], w.wt_q, PW * 2);
  copy_to_lds_async(wl[1], w.wt_k, PW * 2);
  copy_to_lds_async(wl[2], w.wt_v, PW * 2);
  copy_to_lds_async(wl[3], w.wt_g, PW * 2);
  for (int t = threadIdx.x; t < H * C; t += blockDim.x) wbl[t] = w.wb_raw[t];
  for (int t = threadIdx.x; t < C; t += blockDim.x) lnw[t] = w.ln_w[t];
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();

  const int lane = threadIdx.x & 63, half = lane >> 5, t32 = lane & 31;
  const int wave = wave_id();
  bf16* const sw = cst[wave];
  const int jtiles = np / 32;
  const int64_t pitch = bf.pitch;
  const bf16* src[3] = {bf.dq, bf.dk, bf.dv};
  // channel-major planes through descriptors based at the tile's first
  // position, per-lane offsets 32-bit and a channel's offset in the scalar
  // operand (the host checks the ranges fit)
  const uint32_t svo = cm_store_voff(pitch), lvo = cm_load_voff(pitch);
  const uint32_t evo = (uint32_t)(4 * half * pitch + t32) * 2;  // element path: channel 4*half, position t32
  for (int64_t tile = (int64_t)blockIdx.x * 8 + wave; tile < ntiles; tile += (int64_t)gridDim.x * 8) {
    // tile coordinates through readfirstlane: the 64-bit divisions run on the
    // VALU, and descriptors built from their results would otherwise sit in
    // VGPRs, each buffer access in a waterfall loop
    const int jt = __builtin_amdgcn_readfirstlane((int)(tile % jtiles));
    const int r = __builtin_amdgcn_readfirstlane((int)((tile / jtiles) % N));
    const int b = __builtin_amdgcn_readfirstlane((int)(tile / ((int64_t)jtiles * N)));
    const int j = jt * 32 + t32;
    const bool valid = j < N;
    const int64_t xp = valid ? ((int64_t)b * N + (starting ? r : j)) * N + (starting ? j : r) : 0;
    const int64_t p = ((int64_t)b * N + r) * N + j;
    const int64_t p0 = ((int64_t)b * N + r) * N + jt * 32;
    const bool fast = jt * 32 + 32 <= N && N % 8 == 0;  // wave-uniform
    const uint32_t eoff = valid ? evo : kBufSkip;  // stores of padded lanes are dropped
    // per-tile LDS reads of W_b and the LayerNorm weight through an opaque
    // index: hoisted out of the tile loop, 320 of them would stay in registers
    const int oz = opaque_zero();
    const auto srs = buf_rsrc_u(bf.cm_stack + p0, (uint32_t)(4 * CH * pitch * 2));

    f32x2 st;
    {
      RowHalf<C> rhx;
      load_row_half<bf16, C>(rhx, x + xp * C, valid);
      st = row_stats<C>(rhx, eps);
    }
    f32x16 dzn[C / 32];
#pragma unroll
    for (int nt = 0; nt < C / 32; ++nt) dzn[nt] = zero16();
#pragma unroll 1
    for (int kind = 0; kind < 4; ++kind) {
#pragma unroll 1
      for (int h = 0; h < H; ++h) {
        float d[16];
        const uint32_t soff = (uint32_t)((kind * CH + h * AD) * pitch * 2);
        if (kind < 3) {
          const bf16* s = src[kind] + ((((int64_t)b * N + r) * H + h) * np + j) * AD;
#pragma unroll
          for (int g = 0; g < 4; ++g) {
            const f32x4 v4 = load4f(s + 8 * g + 4 * half);
#pragma unroll
            for (int e = 0; e < 4; ++e) d[4 * g + e] = valid ? v4[e] : 0.f;
          }
          if (fast) {
            cm_store_tile(sw, d, srs, svo, soff, pitch);
          } else {
#pragma unroll
            for (int g = 0; g < 4; ++g)
#pragma unroll
              for (int e = 0; e < 4; ++e)
                buf_store_bf16(srs, eoff, soff + (uint32_t)((8 * g + e) * pitch * 2), d[4 * g + e]);
          }
        } else if (fast) {
          cm_load_tile(sw, d, srs, lvo, soff, pitch);
        } else {
          // padded lanes read past the row (or past the range: 0) and are zeroed
#pragma unroll
          for (int g = 0; g < 4; ++g)
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              const float v = buf_load_bf16(srs, evo, soff + (uint32_t)((8 * g + e) * pitch * 2));
              d[4 * g + e] = valid ? v : 0.f;
            }
        }
        Frag<bf16> f[2];
        vals_to_frags<bf16>(f, d);
#pragma unroll
        for (int nt2 = 0; nt2 < C / 32; ++nt2)
#pragma unroll
          for (int gp = 0; gp < 2; ++gp) {
            Frag<bf16> wf;
            load_wfrag_lds(wf, wl[kind], nt2, 2 * h + gp, CH / 16);
            mma(dzn[nt2], wf, f[gp]);
          }
      }
    }
    // triangle bias: dxn += sum_h dB[h][r][j] W_b[h][.]
    float dtri[H];
#pragma unroll
    for (int h = 0; h < H; ++h) {
      dtri[h] = valid ? bf.db[(((int64_t)b * H + h) * N + r) * N + j] : 0.f;
      if (valid && half == 0) bf.cm_dtri[(int64_t)h * pitch + p] = (bf16)dtri[h];
    }
    float s1 = 0.f, s2 = 0.f;
#pragma unroll
    for (int nt = 0; nt < C / 32; ++nt)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int c0 = nt * 32 + 8 * g + 4 * half;
        const f32x4 x4 = load4f(x + xp * C + c0);  // padded lanes: pair 0, their t is 0
        const f32x4 lw = *reinterpret_cast<const f32x4*>(lnw + c0 + oz);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          float t = dzn[nt][4 * g + e];
#pragma unroll
          for (int h = 0; h < H; ++h) t += dtri[h] * wbl[h * C + c0 + e + oz];
          dzn[nt][4 * g + e] = t;
          const float xv = (x4[e] - st[0]) * st[1];
          const float dxh = lw[e] * t;
          s1 += dxh;
          s2 += dxh * xv;
        }
      }
    s1 += xor32(s1);
    s2 += xor32(s2);
    const float m1 = s1 * (1.0f / C), m2 = s2 * (1.0f / C);
    // the rows are read again below rather than kept
    asm volatile("" ::: "memory");
    const auto xrs = buf_rsrc_u(bf.cm_xh + p0, (uint32_t)(C * pitch * 2));
    const auto nrs = buf_rsrc_u(bf.cm_dxn + p0, (uint32_t)(C * pitch * 2));
#pragma unroll
    for (int nt = 0; nt < C / 32; ++nt) {
      float xs[16], dn[16];
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int c0 = nt * 32 + 8 * g + 4 * half;
        const f32x4 x4 = load4f(x + xp * C + c0);  // padded lanes: pair 0, their t is 0
        const f32x4 lw = *reinterpret_cast<const f32x4*>(lnw + c0 + oz);
        float o[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const float xv = (x4[e] - st[0]) * st[1];
          const float t = dzn[nt][4 * g + e];
          o[e] = st[1] * (lw[e] * t - m1 - xv * m2);
          xs[4 * g + e] = xv;
          dn[4 * g + e] = t;
          if (!fast) {
            const uint32_t so = (uint32_t)((nt * 32 + 8 * g + e) * pitch * 2);
            buf_store_bf16(xrs, eoff, so, xv);
            buf_store_bf16(nrs, eoff, so, t);
          }
        }
        if (valid) store4(dx + xp * C + c0, o[0], o[1], o[2], o[3]);
      }
      if (fast) {
        const uint32_t so = (uint32_t)(nt * 32 * pitch * 2);
        cm_store_tile(sw, xs, xrs, svo, so, pitch);
        cm_store_tile(sw, dn, nrs, svo, so, pitch);
      }
    }
  }
}

// dW_b[h][c] = W3[c][h] gamma[c] + s[h] beta[c]  (W3 = sum_s part[s][c][h]: the
// product's layout [nsplit][Cp][64], Cp = C rounded up to its row tile)
__global__ __launch_bounds__(256) void attn_dwb_finish_kernel(const float* __restrict__ part, int nsplit, int C,
                                                            int Cp, int H, const float* __restrict__ gamma,
                                                            const float* __restrict__ beta,
                                                            const float* __restrict__ sums, float* __restrict__ dst) {
  // 8 outputs x 32 chunks of the splits per block (four loads in flight a
  // thread), partial sums added through LDS
  __shared__ float red[32][8];
  const int o = threadIdx.x & 7, ch = threadIdx.x >> 3;
  const int idx = blockIdx.x * 8 + o;
  const bool live = idx < H * C;
  const int h = live ? idx / C : 0, c = live ? idx % C : 0;
  float acc = 0.f;
  if (live) {
    const float* src = part + (int64_t)c * 64 + h;
    const int64_t step = (int64_t)Cp * 64;
    float a[4] = {0.f, 0.f, 0.f, 0.f};
    int s = ch;
    for (; s + 96 < nsplit; s += 128)
#pragma unroll
      for (int u = 0; u < 4; ++u) a[u] += src[(s + 32 * u) * step];
    for (; s < nsplit; s += 32) a[0] += src[s * step];
    acc = (a[0] + a[1]) + (a[2] + a[3]);
  }
  red[ch][o] = acc;
  __syncthreads();
  if (ch != 0 || !live) return;
  for (int k = 1; k < 32; ++k) acc += red[k][o];
  dst[idx] = acc * gamma[c] + sums[h] * beta[c];
}

// ---------------------------------------------------------------------------
// Workspace
// ---------------------------------------------------------------------------
template <typename T> struct AttnBwdWs {
  AttnBwdW<T> w;
  AttnBwdBufs<T> b;
  float *part1, *part2, *part3, *red, *rs, *sums_stack, *sums_dy, *sums_dxn, *dots_dxn, *sums_dtri;
};

template <typename T>
static AttnBwdWs<T> carve_attn_bwd(Carve& cv, int64_t B, int64_t N, int C, int H) {
  const int CH = H * AD;
  AttnBwdWs<T> a;
  AttnBwdW<T>& w = a.w;
  w.w_q = cv.take<T>(packed_elems(CH, C));
  w.w_k = cv.take<T>(packed_elems(CH, C));
  w.w_v = cv.take<T>(packed_elems(CH, C));
  w.w_g = cv.take<T>(packed_elems(CH, C));
  w.w_b = cv.take<T>(packed_elems(H, C));
  w.b_q = cv.take<float>(CH);
  w.b_k = cv.take<float>(CH);
  w.b_v = cv.take<float>(CH);
  w.b_g = cv.take<float>(CH);
  w.b_b = cv.take<float>(32);
  w.wt_q = cv.take<T>(packed_elems(C, CH));
  w.wt_k = cv.take<T>(packed_elems(C, CH));
  w.wt_v = cv.take<T>(packed_elems(C, CH));
  w.wt_g = cv.take<T>(packed_elems(C, CH));
  w.wt_o = cv.take<T>(packed_elems(CH, C));
  w.wb_raw = cv.take<float>((int64_t)H * C);
  w.ln_w = cv.take<float>(C);
  w.ln_b = cv.take<float>(C);
  AttnBwdBufs<T>& b = a.b;
  const int64_t np = round_up(N, 32);
  const int64_t hp = B * N * H * np * AD;
  T** big[] = {&b.qr, &b.qt, &b.kr, &b.kt, &b.vr, &b.vt, &b.o, &b.dor, &b.dot, &b.dq, &b.dk, &b.dv};
  for (T** t : big) *t = cv.take<T>(hp);
  b.gt = cv.take<T>(B * N * np * CH);
  b.bias = cv.take<T>(B * H * N * N);
  b.biasT = cv.take<float>(B * H * np * np);
  b.biasS = cv.take<float>(B * H * np * np);
  b.kmask = cv.take<float>(B * N * np);
  b.mrow = cv.take<float>(B * N * H * np);
  b.linv = cv.take<float>(B * N * H * np);
  b.dd = cv.take<float>(B * N * H * np);
  b.db = cv.take<float>(B * H * N * N);
  b.dbp = (sizeof(T) == 2 && np <= 512) ? cv.take<float>(B * kDbChunks * H * np * np) : nullptr;
  b.pitch = round_up(B * N * N, 64);
  // operands of the weight-gradient products: rows padded to their tiles
  b.cm_stack = cv.take<T>((int64_t)wgrad_rows(4 * CH) * b.pitch);
  b.cm_xh = cv.take<T>((int64_t)wgrad_rows(C) * b.pitch);
  b.cm_dxn = cv.take<T>(C * b.pitch);
  b.cm_dy = cv.take<T>((int64_t)wgrad_rows(C) * b.pitch);
  b.cm_go = cv.take<T>((int64_t)wgrad_rows(CH) * b.pitch);
  b.cm_dtri = cv.take<T>(64 * b.pitch);
  a.part1 = cv.take<float>(wgrad_part_floats(4 * CH, C, b.pitch));
  a.part2 = cv.take<float>(wgrad_part_floats(C, CH, b.pitch));
  a.part3 = cv.take<float>(wgrad_part_floats(C, 64, b.pitch));
  a.red = cv.take<float>((int64_t)2 * 4 * CH * kRowSegs);
  a.rs = cv.take<float>(std::max(wgrad_rowsum_floats(4 * CH, b.pitch), wgrad_rowsum_floats(C, b.pitch)));
  a.sums_stack = cv.take<float>(4 * CH);
  a.sums_dy = cv.take<float>(C);
  a.sums_dxn = cv.take<float>(C);
  a.dots_dxn = cv.take<float>(C);
  a.sums_dtri = cv.take<float>(64);
  return a;
}

template <typename T>
static int pack_attn_bwd(const gtk_tri_attn_weights* wt, AttnBwdW<T>& w, int C, int H,
                         hipStream_t st) {
  const int CH = H * AD, wd = wt->dtype;
  PackScope batch(st);  // the packing launches issued as 3
  int rc;
  if ((rc = launch_to_f32(w.ln_w, wt->ln_w, wd, C, 1.f, 1.f, st))) return rc;
  if ((rc = launch_to_f32(w.ln_b, wt->ln_b, wd, C, 1.f, 0.f, st))) return rc;
  struct Lin { T* dst; float* bdst; const void* wsrc; const void* bsrc; int out; };
  const Lin lins[5] = {{w.w_q, w.b_q, wt->q_w, nullptr, CH}, {w.w_k, w.b_k, wt->k_w, nullptr, CH},
                       {w.w_v, w.b_v, wt->v_w, nullptr, CH}, {w.w_g, w.b_g, wt->g_w, wt->g_b, CH},
                       {w.w_b, w.b_b, wt->tri_w, nullptr, H}};
  for (const Lin& l : lins) {
    if ((rc = launch_pack<T>(l.dst, l.wsrc, wd, l.out, C, C, 1, 1.f, st, w.ln_w))) return rc;
    if ((rc = launch_fold_bias(l.bdst, l.wsrc, l.bsrc, wd, w.ln_b, l.out, C, C, 1, 1.f, st))) return rc;
  }
  T* wts[4] = {w.wt_q, w.wt_k, w.wt_v, w.wt_g};
  const void* srcs[4] = {wt->q_w, wt->k_w, wt->v_w, wt->g_w};
  for (int k = 0; k < 4; ++k)
    if ((rc = launch_pack_acc<T>(wts[k], srcs[k], wd, C, CH, 1, C, st))) return rc;
  if ((rc = launch_pack<T>(w.wt_o, wt->o_w, wd, CH, C, 1, CH, 1.f, st))) return rc;
  if ((rc = launch_to_f32(w.wb_raw, wt->tri_w, wd, H * C, 1.f, 0.f, st))) return rc;
  return batch.flush();
}

template <typename T, int C, int H>
static int bwd_triattn(const void* x, const float* mask, const void* dy,
                       const gtk_tri_attn_weights* wts, void* dx, const gtk_tri_attn_grads* gr,
                       int64_t B, int64_t N, int starting, float eps, void* ws, hipStream_t st) {
  constexpr int CH = H * AD;
  Carve cv(ws, SIZE_MAX);
  AttnBwdWs<T> a = carve_attn_bwd<T>(cv, B, N, C, H);
  int rc;
  if ((rc = pack_attn_bwd<T>(wts, a.w, C, H, st))) return rc;
  const int np = (int)round_up(N, 32);
  const int64_t P = B * N * N, pitch = a.b.pitch;
  const float scale = 1.0f / sqrtf((float)AD);
  const int64_t rowtiles = B * N * (np / 32);
  const int64_t headtiles = B * N * H * (np / 32);
  const int64_t pairtiles = B * H * (int64_t)(np / 32) * (np / 32);
  GTK_REQUIRE(headtiles / 4 < (1ll << 31) && pairtiles / 4 < (1ll << 31), GTK_EUNSUPPORTED,
              "attention backward grid too large");
  auto g4 = [](int64_t t) { return (unsigned)((t + 3) / 4); };
  // (row, head) kernels of the bf16 path: NPM = np rounded up to 256, 512 or 1024 (0: none)
  int npm = 0;
  if constexpr (std::is_same<T, bf16>::value) npm = np <= 256 ? 256 : np <= 512 ? 512 : np <= 1024 ? 1024 : 0;
  // the d-major copies of q, k, v and dO are read only by the per-tile kernels
  const int dmajor = npm == 0;
  {
    StageTimer timer("triattn_bwd_proj", st);
    if constexpr (std::is_same<T, bf16>::value) {
      if (!dmajor) {
        // 16 waves a block (about 100 registers each): four a SIMD
        const int grid = (int)std::min<int64_t>(device_cus(), (rowtiles + 15) / 16);
        attn_bwd_proj_lds_kernel<C, H, 16><<<grid, 1024, 0, st>>>((const bf16*)x, mask, a.w, a.b, (int)B, (int)N,
                                                                  np, starting, eps, 1.0f / scale, rowtiles);
      }
    }
    if (!std::is_same<T, bf16>::value || dmajor)
      attn_bwd_proj_kernel<T, C, H><<<g4(rowtiles), 256, 0, st>>>(
          (const T*)x, mask, a.w, a.b, (int)B, (int)N, np, starting, eps, 1.0f / scale, dmajor);
    GTK_LAUNCH_CHECK();
  }
  const int64_t rblocks = B * N * H;
  GTK_REQUIRE(rblocks < (1ll << 31), GTK_EUNSUPPORTED, "attention backward grid too large");
  auto rh_launch = [&](auto kern256, auto kern512, auto kern1024) {
    auto k = npm == 256 ? kern256 : npm == 512 ? kern512 : kern1024;
    k<<<(unsigned)rblocks, 64 * kRhWaves, 0, st>>>(a.b, (int)B, (int)N, np, scale);
  };
  {
    StageTimer timer("triattn_bwd_fwd", st);
    if constexpr (std::is_same<T, bf16>::value) {
      if (npm) {
        // GENIE_TK_EXACT_SOFTMAX=1: the exact online softmax for every query
        // tile (for tests; otherwise only where the pass without a running
        // maximum leaves its range)
        const char* ex = std::getenv("GENIE_TK_EXACT_SOFTMAX");
        const int exact_only = ex && ex[0] == '1';
        auto k = npm == 256 ? attn_bwd_fwd_rh_kernel<256> : npm == 512 ? attn_bwd_fwd_rh_kernel<512>
                                                                       : attn_bwd_fwd_rh_kernel<1024>;
        k<<<(unsigned)rblocks, 64 * kRhWaves, 0, st>>>(a.b, (int)B, (int)N, np, scale, exact_only);
      } else {
        attn_bwd_fwd_kernel<T, H><<<g4(headtiles), 256, 0, st>>>(a.b, (int)B, (int)N, np, scale);
      }
    } else {
      attn_bwd_fwd_kernel<T, H><<<g4(headtiles), 256, 0, st>>>(a.b, (int)B, (int)N, np, scale);
    }
    GTK_LAUNCH_CHECK();
  }
  {
    StageTimer timer("triattn_bwd_epi", st);
    attn_bwd_epi_kernel<T, C, H><<<g4(rowtiles), 256, 0, st>>>((const T*)dy, a.w, a.b, (int)B,
                                                                (int)N, np, starting, dmajor);
    GTK_LAUNCH_CHECK();
  }
  bool rh_done = false;
  if constexpr (std::is_same<T, bf16>::value) {
    if (npm) {
      {
        StageTimer timer("triattn_bwd_dkdv", st);
        rh_launch(attn_bwd_dkdv_rh_kernel<256>, attn_bwd_dkdv_rh_kernel<512>, attn_bwd_dkdv_rh_kernel<1024>);
        GTK_LAUNCH_CHECK();
      }
      {
        StageTimer timer("triattn_bwd_dq", st);
        rh_launch(attn_bwd_dq_rh_kernel<256>, attn_bwd_dq_rh_kernel<512>, attn_bwd_dq_rh_kernel<1024>);
        GTK_LAUNCH_CHECK();
      }
      rh_done = true;
    }
  }
  if (!rh_done) {
    {
      StageTimer timer("triattn_bwd_dkdv", st);
      attn_bwd_dkdv_kernel<T, H><<<g4(headtiles), 256, 0, st>>>(a.b, (int)B, (int)N, np, scale);
      GTK_LAUNCH_CHECK();
    }
    {
      StageTimer timer("triattn_bwd_dq", st);
      attn_bwd_dq_kernel<T, H><<<g4(headtiles), 256, 0, st>>>(a.b, (int)B, (int)N, np, scale);
      GTK_LAUNCH_CHECK();
    }
  }
  {
    StageTimer timer("triattn_bwd_dbias", st);
    if (a.b.dbp) {
      if constexpr (std::is_same<T, bf16>::value) {
        // row chunks of rpc rows (at most kDbChunks per batch element), partial
        // sums in fragment order, then the sum over the chunks
        const int rpc = (int)((N + kDbChunks - 1) / kDbChunks);
        const int nch = (int)((N + rpc - 1) / rpc);
        const int64_t dblocks = B * nch * H * (((N + 31) / 32 + kDbQt - 1) / kDbQt);
        GTK_REQUIRE(dblocks < (1ll << 31), GTK_EUNSUPPORTED, "attention backward grid too large");
        if (np <= 256)
          attn_bwd_dbias_rh_kernel<256><<<(unsigned)dblocks, 64 * kRhWaves, 0, st>>>(a.b, a.b.dbp, (int)B, (int)N,
                                                                                    np, nch, rpc, scale);
        else
          attn_bwd_dbias_rh_kernel<512><<<(unsigned)dblocks, 64 * kRhWaves, 0, st>>>(a.b, a.b.dbp, (int)B, (int)N,
                                                                                    np, nch, rpc, scale);
        GTK_LAUNCH_CHECK();
        const int64_t rtiles = B * H * (int64_t)(np / 32) * (np / 32);
        attn_bwd_dbias_reduce_kernel<<<(unsigned)rtiles, 256, 0, st>>>(a.b.dbp, a.b.db, (int)B, (int)N, np, nch);
      }
    } else {
      attn_bwd_dbias_kernel<T, H><<<g4(pairtiles), 256, 0, st>>>(a.b, (int)B, (int)N, np, scale);
    }
    GTK_LAUNCH_CHECK();
  }
  // rows H..63 of the dtri operand stay zero
  if ((rc = launch_zero(a.b.cm_dtri + (int64_t)H * pitch, (size_t)(64 - H) * pitch * sizeof(T), st)))
    return rc;
  {
    StageTimer timer("triattn_bwd_pro", st);
    bool lds = false;
    if constexpr (std::is_same<T, bf16>::value) {
      // the LDS kernel addresses cm_stack through 32-bit offsets (N up to
      // about 1440 at B = 1); GENIE_TK_ELEMENT_PATHS=1 selects the
      // element-pointer kernel at any size (for tests)
      const char* ep = std::getenv("GENIE_TK_ELEMENT_PATHS");
      if ((int64_t)4 * CH * pitch * 2 < (1ll << 31) && !(ep && ep[0] == '1')) {
        const int grid = (int)std::min<int64_t>(device_cus(), (rowtiles + 7) / 8);
        attn_bwd_pro_lds_kernel<C, H><<<grid, 512, 0, st>>>((const bf16*)x, (bf16*)dx, a.w, a.b, (int)B,
                                                            (int)N, np, starting, eps, rowtiles);
        lds = true;
      }
    }
    if (!lds)
      attn_bwd_pro_kernel<T, C, H><<<g4(rowtiles), 256, 0, st>>>((const T*)x, (T*)dx, a.w, a.b,
                                                                  (int)B, (int)N, np, starting, eps);
    GTK_LAUNCH_CHECK();
  }
  const AttnBwdBufs<T>& b = a.b;
  if ((rc = launch_zero_tail<T>(b.cm_stack, 4 * CH, pitch, P, st))) return rc;
  if ((rc = launch_zero_tail<T>(b.cm_xh, C, pitch, P, st))) return rc;
  if ((rc = launch_zero_tail<T>(b.cm_dy, C, pitch, P, st))) return rc;
  if ((rc = launch_zero_tail<T>(b.cm_go, CH, pitch, P, st))) return rc;
  if ((rc = launch_zero_tail<T>(b.cm_dtri, H, pitch, P, st))) return rc;
  // LayerNorm parameter gradients straight into the outputs where requested
  auto or_tmp = [](float* dst, float* tmp) { return dst ? dst : tmp; };
  if ((rc = launch_rowred<T>(b.cm_dxn, b.cm_xh, C, pitch, P, a.red, or_tmp(gr->ln_b, a.sums_dxn),
                             or_tmp(gr->ln_w, a.dots_dxn), st)))
    return rc;
  if ((rc = launch_rowred<T>(b.cm_dtri, nullptr, H, pitch, P, a.red, a.sums_dtri, nullptr, st))) return rc;
  // the weight-gradient products also sum their G rows: the bias gradients
  {
    StageTimer timer("triattn_bwd_wgrad", st);
    if ((rc = launch_wgrad<T>(b.cm_stack, b.cm_xh, a.part1, 4 * CH, C, pitch, st, a.rs, a.sums_stack))) return rc;
    if ((rc = launch_wgrad<T>(b.cm_dy, b.cm_go, a.part2, C, CH, pitch, st, a.rs, or_tmp(gr->o_b, a.sums_dy))))
      return rc;
    if ((rc = launch_wgrad<T>(b.cm_xh, b.cm_dtri, a.part3, C, 64, pitch, st))) return rc;
  }
  float* wdst[4] = {gr->q_w, gr->k_w, gr->v_w, gr->g_w};
  WgradSegs wsegs;
  for (int k = 0; k < 4; ++k) wsegs.add(wdst[k], k * CH, CH);
  if ((rc = launch_wgrad_finish(a.part1, 4 * CH, C, pitch, wsegs, a.sums_stack, a.w.ln_w, a.w.ln_b, st)))
    return rc;
  if ((rc = launch_copy_f32(gr->g_b, a.sums_stack + 3 * CH, CH, st))) return rc;
  if ((rc = launch_wgrad_finish(a.part2, C, CH, pitch, 0, C, nullptr, nullptr, nullptr, gr->o_w, st)))
    return rc;
  attn_dwb_finish_kernel<<<(H * C + 7) / 8, 256, 0, st>>>(
      a.part3, wgrad_plan(C, pitch).nsplit, C, wgrad_m_rows(C), H, a.w.ln_w, a.w.ln_b, a.sums_dtri, gr->tri_w);
  GTK_LAUNCH_CHECK();
  return GTK_OK;
}

}  // namespace gtk

using namespace gtk;

// Shapes of the backward kernels: c_in in {32, 64, 128}, four heads of 32
// (modules with fewer or narrower heads pass their weights padded to this).
static bool attn_bwd_shape_ok(int64_t c_in, int64_t c_h, int64_t H) {
  return (c_in == 32 || c_in == 64 || c_in == 128) && H == 4 && c_h == H * AD;
}

template <typename T>
static int bwd_triattn_any(int64_t c_in, const void* x, const float* mask, const void* dy,
                           const gtk_tri_attn_weights* w, void* dx, const gtk_tri_attn_grads* grads,
                           int64_t B, int64_t N, int starting, float eps, void* ws, hipStream_t st) {
  switch (c_in) {
    case 32: return bwd_triattn<T, 32, 4>(x, mask, dy, w, dx, grads, B, N, starting, eps, ws, st);
    case 64: return bwd_triattn<T, 64, 4>(x, mask, dy, w, dx, grads, B, N, starting, eps, ws, st);
    default: return bwd_triattn<T, 128, 4>(x, mask, dy, w, dx, grads, B, N, starting, eps, ws, st);
  }
}

extern "C" size_t gtk_tri_attn_backward_workspace_size(int64_t B, int64_t N, int64_t c_in,
                                                       int64_t c_h, int64_t H, int dtype) {
  if (!attn_bwd_shape_ok(c_in, c_h, H) || B < 0 || N < 0) return 0;
  if (dtype != GTK_F32 && dtype != GTK_BF16) return 0;
  Carve cv(nullptr, SIZE_MAX);
  if (dtype == GTK_F32) carve_attn_bwd<float>(cv, B, N, (int)c_in, (int)H);
  else carve_attn_bwd<bf16>(cv, B, N, (int)c_in, (int)H);
  return cv.off;
}

extern "C" int gtk_tri_attn_backward(const void* x, const float* mask, const void* dy,
                                     const gtk_tri_attn_weights* w, void* dx,
                                     const gtk_tri_attn_grads* grads, int64_t B, int64_t N,
                                     int64_t c_in, int64_t c_h, int64_t H, int starting, float eps,
                                     int dtype, void* ws, size_t ws_bytes, void* stream) {
  GTK_REQUIRE(dtype == GTK_F32 || dtype == GTK_BF16, GTK_EINVAL,
              "gtk_tri_attn_backward: bad dtype %d", dtype);
  GTK_REQUIRE(attn_bwd_shape_ok(c_in, c_h, H), GTK_EUNSUPPORTED,
              "gtk_tri_attn_backward: c_in=%lld c_h=%lld H=%lld unsupported (c_in in {32, 64, 128}, H=4, d=32)",
              (long long)c_in, (long long)c_h, (long long)H);
  GTK_REQUIRE(B >= 0 && N >= 0 && N <= 4096, GTK_EINVAL, "gtk_tri_attn_backward: bad shape");
  if (B == 0 || N == 0) return GTK_OK;
  GTK_REQUIRE(x && dy && w && dx && grads && ws, GTK_EINVAL, "gtk_tri_attn_backward: null pointer");
  GTK_REQUIRE(w->dtype == GTK_F32 || w->dtype == GTK_BF16, GTK_EINVAL,
              "gtk_tri_attn_backward: bad weight dtype %d", w->dtype);
  GTK_REQUIRE(w->tri_w && w->q_w && w->k_w && w->v_w && w->g_w && w->o_w, GTK_EINVAL,
              "gtk_tri_attn_backward: null weight");
  const float* gp[] = {grads->ln_w, grads->ln_b, grads->tri_w, grads->q_w, grads->k_w,
                       grads->v_w,  grads->g_w,  grads->g_b,   grads->o_w, grads->o_b};
  for (const float* p : gp) GTK_REQUIRE(p, GTK_EINVAL, "gtk_tri_attn_backward: null gradient pointer");
  const size_t need = gtk_tri_attn_backward_workspace_size(B, N, c_in, c_h, H, dtype);
  GTK_REQUIRE(ws_bytes >= need, GTK_EWORKSPACE, "gtk_tri_attn_backward: workspace %zu < %zu bytes",
              ws_bytes, need);
  hipStream_t st = (hipStream_t)stream;
  if (dtype == GTK_F32) return bwd_triattn_any<float>(c_in, x, mask, dy, w, dx, grads, B, N, starting, eps, ws, st);
  return bwd_triattn_any<bf16>(c_in, x, mask, dy, w, dx, grads, B, N, starting, eps, ws, st);
}
