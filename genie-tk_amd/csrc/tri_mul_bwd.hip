// Backward of the triangle multiplicative update (outgoing / incoming).
//
// The reference computes gradients with torch autograd over its PyTorch path
// (triangle_mul.py:103-132); this is the same chain rule on the gfx950
// kernels.  Forward activations are recomputed from z, not stored:
//
//  0. pack: the forward's folded weights, and W^T of W_ap, W_ag, W_bp, W_bg,
//     W_g, W_z (unfolded) in accumulator order for the data gradients.
//  1. recompute the A, Bm planes and X = A Bm^T (the forward's kernels).
//  2. epilogue backward, one 32-pair tile per wave:
//       s = sigmoid(g_pre), p = LN_out(x) W_z^T + b_z,   y = s * p
//       dp = dy s,  dg_pre = dy p s (1 - s),  dxn = dp W_z
//       dX = LN_out backward(dxn)            -> dX planes (pair orientation)
//     and dp, dg_pre, x_hat_out, dxn as CM planes (grad_util.hpp).
//  3. contraction backward on the matrix cores, per channel plane:
//       outgoing  dA = dX Bm,       dB = dX^T A
//       incoming  dA^T = Bm^T dX^T, dB^T = A^T dX       (pair orientation)
//     as X = L R^T products of transposed planes.
//  4. prologue backward, one 32-pair tile per wave: the gate algebra of
//     a = m * a_p * sigmoid(a_g) (and b), dzn = sum of the five d_pre W
//     products, dz = LN_in backward(dzn); d_pre, x_hat_in, dzn as CM planes.
//  5. weight gradients: two split-K products over the pairs, row sums for
//     biases and LayerNorm parameters, folded back through gamma and beta.
#include <algorithm>
#include <cstdlib>
#include <type_traits>

#include "capi_util.hpp"
#include "common.hpp"
#include "grad_util.hpp"
#include "pack.hpp"
#include "tri_mul_internal.hpp"

namespace gtk {


// ---------------------------------------------------------------------------
// 2. Epilogue backward.  Tiles cover all Np x Np plane positions so that the
//    padding of the dX planes is written as zero.
// ---------------------------------------------------------------------------
template <typename T, int CZ, int CH, bool FULL = false, bool STGP = true>
__global__ __launch_bounds__(256) void trimul_bwd_epilogue_kernel(
    const T* __restrict__ z, const T* __restrict__ px, const T* __restrict__ dy,
    T* __restrict__ pdx, T* __restrict__ cm_dp, T* __restrict__ cm_dg, T* __restrict__ cm_xo,
    T* __restrict__ cm_dxo, TriMulPacked<T> w, const T* __restrict__ wzt, int B, int N, int Np,
    int64_t pitch, float eps_in, float eps_out) {
  constexpr int XPITCH = CH + 8;
  // bf16 (STGP: the planes' byte offsets fit 32 bits): the dX planes'
  // 32-channel blocks go through a per-wave LDS tile, and for FULL (N % 32 ==
  // 0: every tile is 32 valid pairs on one row) the channel-major blocks too
  constexpr bool STG = sizeof(T) == 2 && STGP;
  static_assert(STG || !FULL, "staged stores are bf16");
  __shared__ __attribute__((aligned(16))) T xs[4][32 * XPITCH];
  __shared__ __attribute__((aligned(16))) bf16 cst[STG ? 4 : 1][STG ? kCmTile : 1];
  const int lane = threadIdx.x & 63;
  const int wave = wave_id();
  bf16* const sw = cst[STG ? wave : 0];
  const int half = lane >> 5;
  const int t32 = lane & 31;
  const int jtiles = Np / 32;
  const int64_t tile = (int64_t)blockIdx.x * 4 + wave;
  if (tile >= (int64_t)B * Np * jtiles) return;
  const int jt = (int)(tile % jtiles);
  const int i = (int)((tile / jtiles) % Np);
  const int b = (int)(tile / ((int64_t)jtiles * Np));
  const int j = jt * 32 + t32;
  const int64_t plane = (int64_t)Np * Np;
  T* dxo = pdx + (int64_t)b * CH * plane + (int64_t)i * Np + j;
  if (i >= N || jt * 32 >= N) {
    for (int c = half * (CH / 2); c < (half + 1) * (CH / 2); ++c) dxo[(int64_t)c * plane] = cvt<T>(0.f);
    return;
  }
  const bool valid = j < N;
  const int64_t pair = ((int64_t)b * N + i) * N + (valid ? j : 0);
  const int64_t pair0 = ((int64_t)b * N + i) * N + jt * 32;

  // gate s = sigmoid(LN_in(z) W_g^T + b_g), accumulator layout
  f32x16 sg[CZ / 32];
  {
    RowHalf<CZ> rh;
    load_row_half<T, CZ>(rh, z + pair * CZ, valid);
    const f32x2 st = row_stats<CZ>(rh, eps_in);
    Frag<T> xf[CZ / 16];
    // the forward's packed weights: LayerNorm affine folded in, or applied here
    if constexpr (trimul_folded<CZ, CH>()) ln_to_frags<T, CZ>(xf, rh, st);
    else ln_affine_to_frags<T, CZ>(xf, rh, st, w.ln_in_w, w.ln_in_b);
#pragma unroll
    for (int nt = 0; nt < CZ / 32; ++nt) {
      sg[nt] = row_gemm_tile<T, CZ, true>(xf, w.w_g, nt);
#pragma unroll
      for (int g = 0; g < 4; ++g)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int c = nt * 32 + 8 * g + 4 * half + r;
          sg[nt][4 * g + r] = gate_from_u(sg[nt][4 * g + r] + w.b_g[c]);
        }
    }
  }

  // x tile X[b][c][i][jt*32 ..] -> LDS [pair][c]
  T* s = xs[wave];
  {
    constexpr int EPC = 16 / sizeof(T);
    constexpr int CPR = 32 / EPC;
    const T* xb = px + (int64_t)b * CH * plane + (int64_t)i * Np + jt * 32;
#pragma unroll 4
    for (int id = lane; id < CH * CPR; id += 64) {
      const int c = id / CPR, part = id % CPR;
      const f32x4 raw = *reinterpret_cast<const f32x4*>(xb + (int64_t)c * plane + part * EPC);
      const T* e = reinterpret_cast<const T*>(&raw);
#pragma unroll
      for (int k = 0; k < EPC; ++k) s[(part * EPC + k) * XPITCH + c] = e[k];
    }
  }
  __builtin_amdgcn_s_waitcnt(0);
  __builtin_amdgcn_wave_barrier();
  RowHalf<CH> xh;
  {
    const T* sr = s + t32 * XPITCH + half * (CH / 2);
#pragma unroll
    for (int ch = 0; ch < CH / 16; ++ch) {
      Frag<T> f;
      f.load(sr + ch * 8);
#pragma unroll
      for (int e = 0; e < 8; ++e) xh.v[ch * 8 + e] = f.get(e);
    }
  }
  const f32x2 so = row_stats<CH>(xh, eps_out);
  Frag<T> yf[CH / 16];
  if constexpr (trimul_folded<CZ, CH>()) ln_to_frags<T, CH>(yf, xh, so);
  else ln_affine_to_frags<T, CH>(yf, xh, so, w.ln_out_w, w.ln_out_b);

  // dp = dy s, dg_pre = dy p s (1 - s)
  Frag<T> dpf[CZ / 16];
#pragma unroll
  for (int nt = 0; nt < CZ / 32; ++nt) {
    const f32x16 pacc = row_gemm_tile<T, CH, true>(yf, w.w_z, nt);
    float dpv[16], dgv[16];
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const int c0 = nt * 32 + 8 * g + 4 * half;
      const f32x4 d4 = valid ? load4f(dy + pair * CZ + c0) : f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const float sv = sg[nt][4 * g + r];
        const float pv = pacc[4 * g + r] + w.b_z[c0 + r];
        dpv[4 * g + r] = d4[r] * sv;
        dgv[4 * g + r] = d4[r] * pv * sv * (1.f - sv);
      }
    }
    if constexpr (FULL) {
      const uint32_t so = (uint32_t)(nt * 32 * pitch) * 2;
      cm_store_tile(sw, dpv, buf_rsrc(cm_dp + pair0, (uint32_t)(CZ * pitch * 2)), cm_store_voff(pitch), so, pitch);
      cm_store_tile(sw, dgv, buf_rsrc(cm_dg + pair0, (uint32_t)(CZ * pitch * 2)), cm_store_voff(pitch), so, pitch);
    } else if (valid) {
#pragma unroll
      for (int g = 0; g < 4; ++g)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int64_t o = (int64_t)(nt * 32 + 8 * g + 4 * half + r) * pitch + pair;
          cm_dp[o] = cvt<T>(dpv[4 * g + r]);
          cm_dg[o] = cvt<T>(dgv[4 * g + r]);
        }
    }
    vals_to_frags<T>(&dpf[2 * nt], dpv);
  }

  // dxn = dp W_z  (outputs over c, accumulator layout)
  f32x16 dxn[CH / 32];
#pragma unroll
  for (int nt = 0; nt < CH / 32; ++nt) {
    dxn[nt] = zero16();
#pragma unroll
    for (int ks = 0; ks < CZ / 16; ++ks) {
      Frag<T> wf;
      load_wfrag<T>(wf, wzt, nt, ks, CZ / 16);
      mma(dxn[nt], wf, dpf[ks]);
    }
  }

  // LayerNorm backward: x_hat from the LDS tile, dx_hat = gamma * dxn
  const T* sr = s + t32 * XPITCH;
  float s1 = 0.f, s2 = 0.f;
#pragma unroll
  for (int nt = 0; nt < CH / 32; ++nt)
#pragma unroll
    for (int g = 0; g < 4; ++g)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int c = nt * 32 + 8 * g + 4 * half + r;
        const float xhat = (to_f32(sr[c]) - so[0]) * so[1];
        const float dxh = w.ln_out_w[c] * dxn[nt][4 * g + r];
        s1 += dxh;
        s2 += dxh * xhat;
      }
  s1 += xor32(s1);
  s2 += xor32(s2);
  const float m1 = s1 * (1.0f / CH), m2 = s2 * (1.0f / CH);
#pragma unroll
  for (int nt = 0; nt < CH / 32; ++nt) {
    float xv[16], dv[16];
#pragma unroll
    for (int g = 0; g < 4; ++g)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int c = nt * 32 + 8 * g + 4 * half + r;
        const float xhat = (to_f32(sr[c]) - so[0]) * so[1];
        const float dxh = w.ln_out_w[c] * dxn[nt][4 * g + r];
        const float dxv = so[1] * (dxh - m1 - xhat * m2);
        xv[4 * g + r] = xhat;
        dv[4 * g + r] = valid ? dxv : 0.f;
        if constexpr (!STG) dxo[(int64_t)c * plane] = cvt<T>(dv[4 * g + r]);
        if constexpr (!FULL) {
          if (valid) {
            cm_xo[(int64_t)c * pitch + pair] = cvt<T>(xhat);
            cm_dxo[(int64_t)c * pitch + pair] = cvt<T>(dxn[nt][4 * g + r]);
          }
        }
      }
    if constexpr (STG) {
      // the tile's 32 plane positions, padding included (written as zero)
      const T* const d0 = pdx + (int64_t)b * CH * plane + (int64_t)i * Np + jt * 32;
      cm_store_tile(sw, dv, buf_rsrc(d0, (uint32_t)(CH * plane * 2)), cm_store_voff(plane),
                    (uint32_t)(nt * 32 * plane) * 2, plane);
    }
    if constexpr (FULL) {
      const uint32_t so2 = (uint32_t)(nt * 32 * pitch) * 2;
      float dn[16];
#pragma unroll
      for (int k = 0; k < 16; ++k) dn[k] = dxn[nt][k];
      cm_store_tile(sw, xv, buf_rsrc(cm_xo + pair0, (uint32_t)(CH * pitch * 2)), cm_store_voff(pitch), so2, pitch);
      cm_store_tile(sw, dn, buf_rsrc(cm_dxo + pair0, (uint32_t)(CH * pitch * 2)), cm_store_voff(pitch), so2, pitch);
    }
  }
}

// ---------------------------------------------------------------------------
// 2b. bf16 epilogue backward for whole tiles (N % 32 == 0) of the shapes whose
//     forward packing folds the LayerNorm affines: the same algebra as the
//     kernel above in persistent 4-wave blocks with W_g, W_z and W_z^T
//     (96 KiB at c_z = c = 128), b_g, b_z and gamma_out in LDS.  The kernel
//     above reads the three matrices from L2 for every 32-pair tile.
// ---------------------------------------------------------------------------
template <int CZ, int CH>
__global__ __launch_bounds__(256) void trimul_bwd_epilogue_lds_kernel(
    const bf16* __restrict__ z, const bf16* __restrict__ px, const bf16* __restrict__ dy,
    bf16* __restrict__ pdx, bf16* __restrict__ cm_dp, bf16* __restrict__ cm_dg, bf16* __restrict__ cm_xo,
    bf16* __restrict__ cm_dxo, TriMulPacked<bf16> w, const bf16* __restrict__ wzt, int B, int N, int Np,
    int64_t pitch, float eps_in, float eps_out, int64_t ntiles) {
  static_assert(trimul_folded<CZ, CH>(), "the LayerNorm affines are in the packed weights");
  constexpr int XPITCH = CH + 8;
  constexpr int PG = CZ * CZ, PZ = CZ * CH;
  __shared__ __attribute__((aligned(1024))) bf16 wl[PG + 2 * PZ];
  __shared__ __attribute__((aligned(16))) bf16 xs[4][32 * XPITCH];
  __shared__ __attribute__((aligned(16))) bf16 cst[4][kCmTile];
  __shared__ __attribute__((aligned(16))) float bl[2 * CZ + CH];
  copy_to_lds_async(wl, w.w_g, PG * 2);
  copy_to_lds_async(wl + PG, w.w_z, PZ * 2);
  copy_to_lds_async(wl + PG + PZ, wzt, PZ * 2);
  for (int t = threadIdx.x; t < CZ; t += blockDim.x) {
    bl[t] = w.b_g[t];
    bl[CZ + t] = w.b_z[t];
  }
  for (int t = threadIdx.x; t < CH; t += blockDim.x) bl[2 * CZ + t] = w.ln_out_w[t];
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  const bf16* const wg = wl;
  const bf16* const wz = wl + PG;
  const bf16* const wzl = wl + PG + PZ;

  const int lane = threadIdx.x & 63;
  const int wave = wave_id();
  bf16* const sw = cst[wave];
  bf16* const s = xs[wave];
  const int half = lane >> 5;
  const int t32 = lane & 31;
  const int jtiles = Np / 32;
  const int64_t plane = (int64_t)Np * Np;
  const uint32_t pvo = cm_store_voff(plane), cvo = cm_store_voff(pitch);
  for (int64_t tile = (int64_t)blockIdx.x * 4 + wave; tile < ntiles; tile += (int64_t)gridDim.x * 4) {
    const int jt = (int)(tile % jtiles);
    const int i = (int)((tile / jtiles) % Np);
    const int b = (int)(tile / ((int64_t)jtiles * Np));
    const int j = jt * 32 + t32;
    // per-tile reads of the LDS vectors through an opaque index (hoisted out
    // of the tile loop they would stay in registers)
    const int oz = opaque_zero();
    const bf16* const d0 = pdx + (int64_t)b * CH * plane + (int64_t)i * Np + jt * 32;
    const auto drs = buf_rsrc(d0, (uint32_t)(CH * plane * 2));
    if (i >= N || jt * 32 >= N) {
      // padding positions of the dX planes: zero
      float zf[16];
#pragma unroll
      for (int k = 0; k < 16; ++k) zf[k] = 0.f;
#pragma unroll
      for (int nt = 0; nt < CH / 32; ++nt) cm_store_tile(sw, zf, drs, pvo, (uint32_t)(nt * 32 * plane) * 2, plane);
      continue;
    }
    const int64_t pair = ((int64_t)b * N + i) * N + j;  // every pair of the tile is valid
    const int64_t pair0 = ((int64_t)b * N + i) * N + jt * 32;

    // gate s = sigmoid(LN_in(z) W_g^T + b_g), accumulator layout
    f32x16 sg[CZ / 32];
    {
      RowHalf<CZ> rh;
      load_row_half<bf16, CZ>(rh, z + pair * CZ, true);
      const f32x2 st = row_stats<CZ>(rh, eps_in);
      Frag<bf16> xf[CZ / 16];
      ln_to_frags<bf16, CZ>(xf, rh, st);
#pragma unroll
      for (int nt = 0; nt < CZ / 32; ++nt) {
        f32x16 acc = zero16();
#pragma unroll
        for (int ks = 0; ks < CZ / 16; ++ks) {
          Frag<bf16> wf;
          load_wfrag_lds(wf, wg, nt, ks, CZ / 16);
          mma(acc, wf, xf[ks]);
        }
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const f32x4 bg = *reinterpret_cast<const f32x4*>(bl + nt * 32 + 8 * g + 4 * half + oz);
#pragma unroll
          for (int r = 0; r < 4; ++r) acc[4 * g + r] = gate_from_u(acc[4 * g + r] + bg[r]);
        }
        sg[nt] = acc;
      }
    }

    // x tile X[b][c][i][jt*32 ..] -> LDS [pair][c]
    {
      constexpr int CPR = 4;  // 16-byte chunks of a channel's 32 pairs
      const bf16* xb = px + (int64_t)b * CH * plane + (int64_t)i * Np + jt * 32;
#pragma unroll 4
      for (int id = lane; id < CH * CPR; id += 64) {
        const int c = id / CPR, part = id % CPR;
        const f32x4 raw = *reinterpret_cast<const f32x4*>(xb + (int64_t)c * plane + part * 8);
        const bf16* e = reinterpret_cast<const bf16*>(&raw);
#pragma unroll
        for (int k = 0; k < 8; ++k) s[(part * 8 + k) * XPITCH + c] = e[k];
      }
    }
    __builtin_amdgcn_s_waitcnt(0);
    __builtin_amdgcn_wave_barrier();
    RowHalf<CH> xh;
    {
      const bf16* sr = s + t32 * XPITCH + half * (CH / 2);
#pragma unroll
      for (int ch = 0; ch < CH / 16; ++ch) {
        Frag<bf16> f;
        f.load(sr + ch * 8);
#pragma unroll
        for (int e = 0; e < 8; ++e) xh.v[ch * 8 + e] = f.get(e);
      }
    }
    const f32x2 so = row_stats<CH>(xh, eps_out);
    Frag<bf16> yf[CH / 16];
    ln_to_frags<bf16, CH>(yf, xh, so);

    // dp = dy s, dg_pre = dy p s (1 - s)
    Frag<bf16> dpf[CZ / 16];
    const auto prs = buf_rsrc(cm_dp + pair0, (uint32_t)(CZ * pitch * 2));
    const auto grs = buf_rsrc(cm_dg + pair0, (uint32_t)(CZ * pitch * 2));
#pragma unroll
    for (int nt = 0; nt < CZ / 32; ++nt) {
      f32x16 pacc = zero16();
#pragma unroll
      for (int ks = 0; ks < CH / 16; ++ks) {
        Frag<bf16> wf;
        load_wfrag_lds(wf, wz, nt, ks, CH / 16);
        mma(pacc, wf, yf[ks]);
      }
      float dpv[16], dgv[16];
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int c0 = nt * 32 + 8 * g + 4 * half;
        const f32x4 d4 = load4f(dy + pair * CZ + c0);
        const f32x4 bz = *reinterpret_cast<const f32x4*>(bl + CZ + c0 + oz);
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const float sv = sg[nt][4 * g + r];
          const float pv = pacc[4 * g + r] + bz[r];
          dpv[4 * g + r] = d4[r] * sv;
          dgv[4 * g + r] = d4[r] * pv * sv * (1.f - sv);
        }
      }
      const uint32_t so2 = (uint32_t)(nt * 32 * pitch) * 2;
      cm_store_tile(sw, dpv, prs, cvo, so2, pitch);
      cm_store_tile(sw, dgv, grs, cvo, so2, pitch);
      vals_to_frags<bf16>(&dpf[2 * nt], dpv);
    }

    // dxn = dp W_z  (outputs over c, accumulator layout)
    f32x16 dxn[CH / 32];
#pragma unroll
    for (int nt = 0; nt < CH / 32; ++nt) {
      dxn[nt] = zero16();
#pragma unroll
      for (int ks = 0; ks < CZ / 16; ++ks) {
        Frag<bf16> wf;
        load_wfrag_lds(wf, wzl, nt, ks, CZ / 16);
        mma(dxn[nt], wf, dpf[ks]);
      }
    }

    // LayerNorm backward: x_hat from the LDS tile, dx_hat = gamma * dxn
    const bf16* sr = s + t32 * XPITCH;
    float s1 = 0.f, s2 = 0.f;
#pragma unroll
    for (int nt = 0; nt < CH / 32; ++nt)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int c0 = nt * 32 + 8 * g + 4 * half;
        const f32x4 lw = *reinterpret_cast<const f32x4*>(bl + 2 * CZ + c0 + oz);
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const float xhat = (to_f32(sr[c0 + r]) - so[0]) * so[1];
          const float dxh = lw[r] * dxn[nt][4 * g + r];
          s1 += dxh;
          s2 += dxh * xhat;
        }
      }
    s1 += xor32(s1);
    s2 += xor32(s2);
    const float m1 = s1 * (1.0f / CH), m2 = s2 * (1.0f / CH);
    const auto xrs = buf_rsrc(cm_xo + pair0, (uint32_t)(CH * pitch * 2));
    const auto nrs = buf_rsrc(cm_dxo + pair0, (uint32_t)(CH * pitch * 2));
#pragma unroll
    for (int nt = 0; nt < CH / 32; ++nt) {
      float xv[16], dv[16], dn[16];
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int c0 = nt * 32 + 8 * g + 4 * half;
        const f32x4 lw = *reinterpret_cast<const f32x4*>(bl + 2 * CZ + c0 + oz);
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const float xhat = (to_f32(sr[c0 + r]) - so[0]) * so[1];
          const float dxh = lw[r] * dxn[nt][4 * g + r];
          xv[4 * g + r] = xhat;
          dv[4 * g + r] = so[1] * (dxh - m1 - xhat * m2);
          dn[4 * g + r] = dxn[nt][4 * g + r];
        }
      }
      cm_store_tile(sw, dv, drs, pvo, (uint32_t)(nt * 32 * plane) * 2, plane);
      const uint32_t so2 = (uint32_t)(nt * 32 * pitch) * 2;
      cm_store_tile(sw, xv, xrs, cvo, so2, pitch);
      cm_store_tile(sw, dn, nrs, cvo, so2, pitch);
    }
  }
}

// ---------------------------------------------------------------------------
// 4. Prologue backward.  Tiles over valid rows; da/db planes in pair
//    orientation [b][c][i][j].
// ---------------------------------------------------------------------------
template <typename T, int CZ, int CH>
__global__ __launch_bounds__(256) void trimul_bwd_prologue_kernel(
    const T* __restrict__ z, const float* __restrict__ mask, const T* __restrict__ pda,
    const T* __restrict__ pdb, T* __restrict__ dz, T* __restrict__ cm_stack,
    T* __restrict__ cm_xi, T* __restrict__ cm_dzn, TriMulPacked<T> w, const T* __restrict__ wt,
    const T* __restrict__ wgt, int B, int N, int Np, int64_t pitch, float eps_in) {
  constexpr int64_t PE = (CZ / 32) * (CH / 16) * 512;  // packed_elems(CZ, CH)
  const int lane = threadIdx.x & 63;
  const int wave = wave_id();
  const int half = lane >> 5;
  const int t32 = lane & 31;
  const int jtiles = (N + 31) / 32;
  const int64_t tile = (int64_t)blockIdx.x * 4 + wave;
  if (tile >= (int64_t)B * N * jtiles) return;
  const int jt = (int)(tile % jtiles);
  const int i = (int)((tile / jtiles) % N);
  const int b = (int)(tile / ((int64_t)jtiles * N));
  const int j = jt * 32 + t32;
  const bool valid = j < N;
  const int64_t pair = ((int64_t)b * N + i) * N + (valid ? j : 0);
  const int64_t plane = (int64_t)Np * Np;

  RowHalf<CZ> rh;
  load_row_half<T, CZ>(rh, z + pair * CZ, valid);
  const f32x2 st = row_stats<CZ>(rh, eps_in);
  Frag<T> xf[CZ / 16];
  if constexpr (trimul_folded<CZ, CH>()) ln_to_frags<T, CZ>(xf, rh, st);
  else ln_affine_to_frags<T, CZ>(xf, rh, st, w.ln_in_w, w.ln_in_b);
  const float m = valid ? (mask ? mask[pair] : 1.0f) : 0.0f;

  f32x16 dzn[CZ / 32];
#pragma unroll
  for (int nt = 0; nt < CZ / 32; ++nt) dzn[nt] = zero16();

#pragma unroll 1
  for (int side = 0; side < 2; ++side) {
    const T* wp = side ? w.w_bp : w.w_ap;
    const T* wg = side ? w.w_bg : w.w_ag;
    const float* bp = side ? w.b_bp : w.b_ap;
    const float* bg = side ? w.b_bg : w.b_ag;
    const T* src = (side ? pdb : pda) + (int64_t)b * CH * plane + (int64_t)i * Np + j;
    const T* wtp = wt + (2 * side) * PE;
    const T* wtg = wt + (2 * side + 1) * PE;
    T* cm_p = cm_stack + (int64_t)(2 * side) * CH * pitch;
    T* cm_g = cm_stack + (int64_t)(2 * side + 1) * CH * pitch;
#pragma unroll 1
    for (int nt = 0; nt < CH / 32; ++nt) {
      const f32x16 pre = row_gemm_tile<T, CZ, true>(xf, wp, nt);
      const f32x16 u = row_gemm_tile<T, CZ, true>(xf, wg, nt);
      float d_p[16], d_g[16];
#pragma unroll
      for (int g = 0; g < 4; ++g)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int c = nt * 32 + 8 * g + 4 * half + r;
          const float v = pre[4 * g + r] + bp[c];
          const float sv = gate_from_u(u[4 * g + r] + bg[c]);
          const float d = valid ? to_f32(src[(int64_t)c * plane]) * m : 0.f;
          d_p[4 * g + r] = d * sv;
          d_g[4 * g + r] = d * v * sv * (1.f - sv);
        }
      if (valid) {
#pragma unroll
        for (int g = 0; g < 4; ++g)
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const int64_t o = (int64_t)(nt * 32 + 8 * g + 4 * half + r) * pitch + pair;
            cm_p[o] = cvt<T>(d_p[4 * g + r]);
            cm_g[o] = cvt<T>(d_g[4 * g + r]);
          }
      }
      Frag<T> fp[2], fg[2];
      vals_to_frags<T>(fp, d_p);
      vals_to_frags<T>(fg, d_g);
#pragma unroll
      for (int nt2 = 0; nt2 < CZ / 32; ++nt2)
#pragma unroll
        for (int gp = 0; gp < 2; ++gp) {
          Frag<T> wf;
          load_wfrag<T>(wf, wtp, nt2, 2 * nt + gp, CH / 16);
          mma(dzn[nt2], wf, fp[gp]);
          load_wfrag<T>(wf, wtg, nt2, 2 * nt + gp, CH / 16);
          mma(dzn[nt2], wf, fg[gp]);
        }
    }
  }
  // the output gate's share: dg_pre W_g
  {
    const T* cm_dg = cm_stack + (int64_t)4 * CH * pitch;
#pragma unroll 1
    for (int nt = 0; nt < CZ / 32; ++nt) {
      float d[16];
#pragma unroll
      for (int g = 0; g < 4; ++g)
#pragma unroll
        for (int r = 0; r < 4; ++r)
          d[4 * g + r] = valid ? to_f32(cm_dg[(int64_t)(nt * 32 + 8 * g + 4 * half + r) * pitch + pair]) : 0.f;
      Frag<T> f[2];
      vals_to_frags<T>(f, d);
#pragma unroll
      for (int nt2 = 0; nt2 < CZ / 32; ++nt2)
#pragma unroll
        for (int gp = 0; gp < 2; ++gp) {
          Frag<T> wf;
          load_wfrag<T>(wf, wgt, nt2, 2 * nt + gp, CZ / 16);
          mma(dzn[nt2], wf, f[gp]);
        }
    }
  }

  // LayerNorm backward in accumulator layout
  float xh[CZ / 2];
  float s1 = 0.f, s2 = 0.f;
#pragma unroll
  for (int nt = 0; nt < CZ / 32; ++nt)
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const int c0 = nt * 32 + 8 * g + 4 * half;
      const f32x4 z4 = valid ? load4f(z + pair * CZ + c0) : f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const float xv = (z4[r] - st[0]) * st[1];
        xh[16 * nt + 4 * g + r] = xv;
        const float dxh = w.ln_in_w[c0 + r] * dzn[nt][4 * g + r];
        s1 += dxh;
        s2 += dxh * xv;
      }
    }
  s1 += xor32(s1);
  s2 += xor32(s2);
  const float m1 = s1 * (1.0f / CZ), m2 = s2 * (1.0f / CZ);
  if (!valid) return;
#pragma unroll
  for (int nt = 0; nt < CZ / 32; ++nt)
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const int c0 = nt * 32 + 8 * g + 4 * half;
      float o[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const float xv = xh[16 * nt + 4 * g + r];
        const float dxh = w.ln_in_w[c0 + r] * dzn[nt][4 * g + r];
        o[r] = st[1] * (dxh - m1 - xv * m2);
        cm_xi[(int64_t)(c0 + r) * pitch + pair] = cvt<T>(xv);
        cm_dzn[(int64_t)(c0 + r) * pitch + pair] = cvt<T>(dzn[nt][4 * g + r]);
      }
      store4(dz + pair * CZ + c0, o[0], o[1], o[2], o[3]);
    }
}

// ---------------------------------------------------------------------------
// 4b. bf16 prologue backward, one launch per side.  The kernel above reads
//     every weight fragment of its matrix products from L2 (about 256 KiB a
//     32-pair tile) at one wave per SIMD (over 400 registers), and waits on
//     each.  Here each launch keeps one side's forward and transposed
//     weights (4 x c x c_z bf16, 128 KiB at c_z = c = 128) in LDS, and the
//     blocks are persistent, 8 waves (two a SIMD, at most 256 registers).  SIDE 0 (a) writes its share of dL/dzn as an
//     fp32 partial in the accumulator layout ([tile][c_z / 32][4][64 lanes]
//     x 4 floats, 1 KiB contiguous a store), with the output gate's share
//     (dg_pre W_g, W_g^T from L2) added; SIDE 1 (b) adds its own share and
//     runs the LayerNorm backward.
// ---------------------------------------------------------------------------
template <int CZ, int CH, int SIDE, bool FULL>
__global__ __launch_bounds__(512) void trimul_bwd_prologue_side_kernel(
    const bf16* __restrict__ z, const float* __restrict__ mask, const bf16* __restrict__ pd,
    bf16* __restrict__ dz, bf16* __restrict__ cm_stack, bf16* __restrict__ cm_xi,
    bf16* __restrict__ cm_dzn, TriMulPacked<bf16> w, const bf16* __restrict__ wt,
    const bf16* __restrict__ wgt, float* __restrict__ part, int B, int N, int Np, int64_t pitch,
    float eps_in, int64_t ntiles) {
  constexpr int PW = CH * CZ;  // elements of one packed c_z x c weight
  // [0] W_p, [1] W_g of this side (forward, the kernels' packing, folded as
  // the forward's); [2] W_p^T, [3] W_g^T (raw, accumulator packing)
  __shared__ __attribute__((aligned(1024))) bf16 wl[4][PW];
  copy_to_lds_async(wl[0], SIDE ? w.w_bp : w.w_ap, PW * 2);
  copy_to_lds_async(wl[1], SIDE ? w.w_bg : w.w_ag, PW * 2);
  copy_to_lds_async(wl[2], wt + (int64_t)(2 * SIDE) * PW, PW * 2);
  copy_to_lds_async(wl[3], wt + (int64_t)(2 * SIDE + 1) * PW, PW * 2);
  // FULL (N % 32 == 0): every tile is 32 valid pairs on one row, and the
  // channel-major blocks go through a per-wave LDS tile
  __shared__ __attribute__((aligned(16))) bf16 cst[FULL ? 8 : 1][FULL ? kCmTile : 1];
  // this side's biases and the LayerNorm weight: read per tile from LDS, so
  // that no global load of theirs makes a stage wait for every load in flight
  __shared__ __attribute__((aligned(16))) float bl[2 * CH + CZ];
  for (int t = threadIdx.x; t < CH; t += blockDim.x) {
    bl[t] = (SIDE ? w.b_bp : w.b_ap)[t];
    bl[CH + t] = (SIDE ? w.b_bg : w.b_ag)[t];
  }
  for (int t = threadIdx.x; t < CZ; t += blockDim.x) bl[2 * CH + t] = w.ln_in_w[t];
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();

  const int lane = threadIdx.x & 63;
  const int wave = wave_id();
  bf16* const sw = cst[FULL ? wave : 0];
  const int half = lane >> 5;
  const int t32 = lane & 31;
  const int jtiles = (N + 31) / 32;
  const int64_t plane = (int64_t)Np * Np;
  const float* const bp = bl;
  const float* const bg = bl + CH;
  const float* const lnw = bl + 2 * CH;
  bf16* const cm_p = cm_stack + (int64_t)(2 * SIDE) * CH * pitch;
  bf16* const cm_g = cm_stack + (int64_t)(2 * SIDE + 1) * CH * pitch;

  for (int64_t tile = (int64_t)blockIdx.x * 8 + wave; tile < ntiles; tile += (int64_t)gridDim.x * 8) {
    const int jt = (int)(tile % jtiles);
    const int i = (int)((tile / jtiles) % N);
    const int b = (int)(tile / ((int64_t)jtiles * N));
    const int j = jt * 32 + t32;
    const bool valid = j < N;
    const int64_t pair = ((int64_t)b * N + i) * N + (valid ? j : 0);
    const int oz = opaque_zero();

    RowHalf<CZ> rh;
    load_row_half<bf16, CZ>(rh, z + pair * CZ, valid);
    const f32x2 st = row_stats<CZ>(rh, eps_in);
    Frag<bf16> xf[CZ / 16];
    if constexpr (trimul_folded<CZ, CH>()) ln_to_frags<bf16, CZ>(xf, rh, st);
    else ln_affine_to_frags<bf16, CZ>(xf, rh, st, w.ln_in_w, w.ln_in_b);
    const float m = valid ? (mask ? mask[pair] : 1.0f) : 0.0f;

    // this tile's partial: [c_z / 32][4 groups][64 lanes] x f32x4
    float* const pt = part + tile * (int64_t)(CZ * 64);
    f32x16 dzn[CZ / 32];
#pragma unroll
    for (int nt = 0; nt < CZ / 32; ++nt) {
      if constexpr (SIDE == 0) {
        dzn[nt] = zero16();
      } else {
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const f32x4 v = *reinterpret_cast<const f32x4*>(pt + ((nt * 4 + g) * 64 + lane) * 4);
#pragma unroll
          for (int r = 0; r < 4; ++r) dzn[nt][4 * g + r] = v[r];
        }
      }
    }

    // the dA / dB planes and the CM planes through descriptors whose bases
    // are the tile's first pair (wave-uniform) and whose per-lane offsets are
    // 32-bit (the host checks the ranges fit); lanes past N store nothing
    const int64_t pair0 = ((int64_t)b * N + i) * N + jt * 32;
    const auto srs = buf_rsrc(pd + (int64_t)b * CH * plane + (int64_t)i * Np + jt * 32,
                              (uint32_t)(CH * plane * 2));
    const auto prs = buf_rsrc(cm_p + pair0, (uint32_t)(CH * pitch * 2));
    const auto grs = buf_rsrc(cm_g + pair0, (uint32_t)(CH * pitch * 2));
    // per-lane byte offsets (channel 4*half, pair t32); the channel offsets
    // of a (nt, g, r) are wave-uniform and go in the scalar operand
    const uint32_t soff = (uint32_t)(4 * half * plane + t32) * 2;
    const uint32_t coff = valid ? (uint32_t)(4 * half * pitch + t32) * 2 : kBufSkip;
#pragma unroll 1
    for (int nt = 0; nt < CH / 32; ++nt) {
      // the forward's pre-activations of channels nt*32 .. +31 (lane = pair)
      f32x16 pre = zero16(), u = zero16();
#pragma unroll
      for (int ks = 0; ks < CZ / 16; ++ks) {
        Frag<bf16> wf;
        load_wfrag_lds(wf, wl[0], nt, ks, CZ / 16);
        mma(pre, wf, xf[ks]);
        load_wfrag_lds(wf, wl[1], nt, ks, CZ / 16);
        mma(u, wf, xf[ks]);
      }
      float d_p[16], d_g[16];
      float dd[16];
      if constexpr (FULL) cm_load_tile(sw, dd, srs, cm_load_voff(plane), (uint32_t)(nt * 32 * plane) * 2, plane);
#pragma unroll
      for (int g = 0; g < 4; ++g)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int c = nt * 32 + 8 * g + 4 * half + r;
          // per-tile reads (opaque index): hoisted out of the tile loop,
          // the 2 x 64 biases of a lane would stay in registers
          const int cx = c + oz;
          const float v = pre[4 * g + r] + bp[cx];
          const float sv = gate_from_u(u[4 * g + r] + bg[cx]);
          const float d = m * (FULL ? dd[4 * g + r]
                                    : buf_load_bf16(srs, soff, (uint32_t)((nt * 32 + 8 * g + r) * plane) * 2));
          d_p[4 * g + r] = d * sv;
          d_g[4 * g + r] = d * v * sv * (1.f - sv);
        }
      if constexpr (FULL) {
        const uint32_t so = (uint32_t)(nt * 32 * pitch) * 2;
        cm_store_tile(sw, d_p, prs, cm_store_voff(pitch), so, pitch);
        cm_store_tile(sw, d_g, grs, cm_store_voff(pitch), so, pitch);
      } else {
#pragma unroll
        for (int g = 0; g < 4; ++g)
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const uint32_t so = (uint32_t)((nt * 32 + 8 * g + r) * pitch) * 2;
            buf_store_bf16(prs, coff, so, d_p[4 * g + r]);
            buf_store_bf16(grs, coff, so, d_g[4 * g + r]);
          }
      }
      Frag<bf16> fp[2], fg[2];
      vals_to_frags<bf16>(fp, d_p);
      vals_to_frags<bf16>(fg, d_g);
#pragma unroll
      for (int nt2 = 0; nt2 < CZ / 32; ++nt2)
#pragma unroll
        for (int gp = 0; gp < 2; ++gp) {
          Frag<bf16> wf;
          load_wfrag_lds(wf, wl[2], nt2, 2 * nt + gp, CH / 16);
          mma(dzn[nt2], wf, fp[gp]);
          load_wfrag_lds(wf, wl[3], nt2, 2 * nt + gp, CH / 16);
          mma(dzn[nt2], wf, fg[gp]);
        }
    }
    // the output gate's share: dg_pre W_g (side a's launch)
    if constexpr (SIDE == 0) {
      const auto drs = buf_rsrc(cm_stack + (int64_t)4 * CH * pitch + pair0, (uint32_t)(CZ * pitch * 2));
#pragma unroll 1
      for (int nt = 0; nt < CZ / 32; ++nt) {
        float d[16];
        if constexpr (FULL) {
          cm_load_tile(sw, d, drs, cm_load_voff(pitch), (uint32_t)(nt * 32 * pitch) * 2, pitch);
        } else {
#pragma unroll
          for (int g = 0; g < 4; ++g)
#pragma unroll
            for (int r = 0; r < 4; ++r)
              d[4 * g + r] = buf_load_bf16(drs, coff, (uint32_t)((nt * 32 + 8 * g + r) * pitch) * 2);
        }
        Frag<bf16> f[2];
        vals_to_frags<bf16>(f, d);
#pragma unroll
        for (int nt2 = 0; nt2 < CZ / 32; ++nt2)
#pragma unroll
          for (int gp = 0; gp < 2; ++gp) {
            Frag<bf16> wf;
            load_wfrag<bf16>(wf, wgt, nt2, 2 * nt + gp, CZ / 16);
            mma(dzn[nt2], wf, f[gp]);
          }
      }
    }
    if constexpr (SIDE == 0) {
#pragma unroll
      for (int nt = 0; nt < CZ / 32; ++nt)
#pragma unroll
        for (int g = 0; g < 4; ++g)
          *reinterpret_cast<f32x4*>(pt + ((nt * 4 + g) * 64 + lane) * 4) =
              f32x4{dzn[nt][4 * g], dzn[nt][4 * g + 1], dzn[nt][4 * g + 2], dzn[nt][4 * g + 3]};
      continue;
    }
    // LayerNorm backward in accumulator layout (x_hat recomputed from z)
    float s1 = 0.f, s2 = 0.f;
#pragma unroll
    for (int nt = 0; nt < CZ / 32; ++nt)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int c0 = nt * 32 + 8 * g + 4 * half;
        const f32x4 z4 = load4f(z + pair * CZ + c0);  // padded lanes: pair j = 0, dzn 0
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const float xv = (z4[r] - st[0]) * st[1];
          const float dxh = lnw[c0 + r + oz] * dzn[nt][4 * g + r];
          s1 += dxh;
          s2 += dxh * xv;
        }
      }
    s1 += xor32(s1);
    s2 += xor32(s2);
    const float m1 = s1 * (1.0f / CZ), m2 = s2 * (1.0f / CZ);
    // the rows are read again below rather than kept (64 values a lane)
    asm volatile("" ::: "memory");
    const auto xrs = buf_rsrc(cm_xi + pair0, (uint32_t)(CZ * pitch * 2));
    const auto nrs = buf_rsrc(cm_dzn + pair0, (uint32_t)(CZ * pitch * 2));
    const auto zrs = buf_rsrc(dz + pair0 * CZ, (uint32_t)(32 * CZ * 2));
    const uint32_t zoff = valid ? (uint32_t)(t32 * CZ) * 2 : kBufSkip;
#pragma unroll
    for (int nt = 0; nt < CZ / 32; ++nt) {
      float xs[16];
      uint32_t pk[4][2];
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int c0 = nt * 32 + 8 * g + 4 * half;
        const f32x4 z4 = load4f(z + pair * CZ + c0);  // padded lanes: pair j = 0, dzn 0
        float o[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const float xv = (z4[r] - st[0]) * st[1];
          const float dxh = lnw[c0 + r + oz] * dzn[nt][4 * g + r];
          o[r] = st[1] * (dxh - m1 - xv * m2);
          xs[4 * g + r] = xv;
          if constexpr (!FULL) {
            const uint32_t so = (uint32_t)((nt * 32 + 8 * g + r) * pitch) * 2;
            buf_store_bf16(xrs, coff, so, xv);
            buf_store_bf16(nrs, coff, so, dzn[nt][4 * g + r]);
          }
        }
        pk[g][0] = pack_bf16x2(o[0], o[1]);
        pk[g][1] = pack_bf16x2(o[2], o[3]);
      }
      // dz leaves as two 16-byte stores a lane: the half-waves trade channel
      // quads (v_permlane32_swap) so that each lane holds 8 consecutive
      // channels of its row
#pragma unroll
      for (int p2 = 0; p2 < 2; ++p2) {
        const auto s0 = __builtin_amdgcn_permlane32_swap(pk[2 * p2][0], pk[2 * p2 + 1][0], false, false);
        const auto s1 = __builtin_amdgcn_permlane32_swap(pk[2 * p2][1], pk[2 * p2 + 1][1], false, false);
        const uint4 c = half ? make_uint4(s0[0], s1[0], pk[2 * p2 + 1][0], pk[2 * p2 + 1][1])
                             : make_uint4(pk[2 * p2][0], pk[2 * p2][1], s0[1], s1[1]);
        buf_store16(zrs, zoff + (uint32_t)(nt * 32 + 16 * p2 + 8 * half) * 2, c);
      }
      if constexpr (FULL) {
        const uint32_t so = (uint32_t)(nt * 32 * pitch) * 2;
        float dn[16];
#pragma unroll
        for (int k = 0; k < 16; ++k) dn[k] = dzn[nt][k];
        cm_store_tile(sw, xs, xrs, cm_store_voff(pitch), so, pitch);
        cm_store_tile(sw, dn, nrs, cm_store_voff(pitch), so, pitch);
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Workspace
// ---------------------------------------------------------------------------
template <typename T> struct TriMulBwdWs {
  void* packed;
  T *wzt, *wt, *wgt;
  T *pa, *pb, *px, *pdx, *pat, *pbt, *pda, *pdb;
  T *cm_stack, *cm_dp, *cm_xi, *cm_xo, *cm_dzn, *cm_dxo;
  float *part1, *part2, *red, *rs, *sums_stack, *sums_dp, *sums_dzn, *dots_dzn, *sums_dxo, *dots_dxo;
  float* part_dzn;  // bf16: side a's share of dL/dzn between the two prologue launches
  int64_t pitch;
};

// Does the contraction backward transpose its planes first?  Only where the
// tile kernels cannot read the operands transposed, or when the test switch
// GENIE_TK_TRANSPOSE_PLANES=1 asks for it (the transposed planes then take
// workspace).
static bool trimul_bwd_transposes(int64_t B, int64_t N, int c, int dtype) {
  const char* tp = std::getenv("GENIE_TK_TRANSPOSE_PLANES");
  if (tp && tp[0] == '1') return true;
  return !trimul_contract_t_ok((int)round_up(N, 64), B * c, dtype);
}

template <typename T>
static TriMulBwdWs<T> carve_trimul_bwd(Carve& cv, int64_t B, int64_t N, int cz, int c, int dtype) {
  TriMulBwdWs<T> w;
  const int64_t Np = round_up(N, 64);
  const int64_t P = B * N * N;
  w.pitch = round_up(P, 64);
  const int M1 = 4 * c + cz;
  w.packed = cv.take<char>((int64_t)gtk_tri_mul_packed_size(cz, c, dtype));
  w.wzt = cv.take<T>(packed_elems(c, cz));
  w.wt = cv.take<T>(4 * packed_elems(cz, c));
  w.wgt = cv.take<T>(packed_elems(cz, cz));
  const int64_t pe = B * c * Np * Np;
  T** planes[] = {&w.pa, &w.pb, &w.px, &w.pdx, &w.pda, &w.pdb};
  for (T** p : planes) *p = cv.take<T>(pe);
  w.pat = w.pbt = nullptr;
  if (trimul_bwd_transposes(B, N, c, dtype)) {
    w.pat = cv.take<T>(pe);
    w.pbt = cv.take<T>(pe);
  }
  // operands of the weight-gradient products: rows padded to their tiles
  w.cm_stack = cv.take<T>((int64_t)wgrad_rows(M1) * w.pitch);
  w.cm_dp = cv.take<T>((int64_t)wgrad_rows(cz) * w.pitch);
  w.cm_xi = cv.take<T>((int64_t)wgrad_rows(cz) * w.pitch);
  w.cm_xo = cv.take<T>((int64_t)wgrad_rows(c) * w.pitch);
  w.cm_dzn = cv.take<T>(cz * w.pitch);
  w.cm_dxo = cv.take<T>(c * w.pitch);
  w.part1 = cv.take<float>(wgrad_part_floats(M1, cz, w.pitch));
  w.part2 = cv.take<float>(wgrad_part_floats(cz, c, w.pitch));
  w.red = cv.take<float>((int64_t)2 * M1 * kRowSegs);
  w.rs = cv.take<float>(std::max(wgrad_rowsum_floats(M1, w.pitch), wgrad_rowsum_floats(cz, w.pitch)));
  w.sums_stack = cv.take<float>(M1);
  w.sums_dp = cv.take<float>(cz);
  w.sums_dzn = cv.take<float>(cz);
  w.dots_dzn = cv.take<float>(cz);
  w.sums_dxo = cv.take<float>(c);
  w.dots_dxo = cv.take<float>(c);
  w.part_dzn = nullptr;
  if constexpr (sizeof(T) == 2) w.part_dzn = cv.take<float>(B * N * ((N + 31) / 32) * (int64_t)cz * 64);
  return w;
}

template <typename T, int CZ, int CH>
static int bwd_trimul(const void* z, const float* mask, const void* dy,
                      const gtk_tri_mul_weights* wts, void* dz, const gtk_tri_mul_grads* gr,
                      int64_t B, int64_t N, int outgoing, float eps_in, float eps_out, int dtype,
                      void* ws, hipStream_t st) {
  Carve cv(ws, SIZE_MAX);
  TriMulBwdWs<T> a = carve_trimul_bwd<T>(cv, B, N, CZ, CH, dtype);
  const int Np = (int)round_up(N, 64);
  const int64_t P = B * N * N, pitch = a.pitch;
  const int64_t nplanes = B * CH;
  const int M1 = 4 * CH + CZ;
  const int wd = wts->dtype;
  int rc;
  // The bf16 kernels' descriptor paths address the channel-major buffers and
  // the dA / dB / dX planes with 32-bit byte offsets; beyond that (N above
  // about 2900 at B = 1) the element-pointer kernels run.  The environment
  // variable GENIE_TK_ELEMENT_PATHS=1 selects them at any size (for tests).
  const char* ep = std::getenv("GENIE_TK_ELEMENT_PATHS");
  const bool fits32 =
      (int64_t)std::max(CZ, CH) * std::max<int64_t>(pitch, (int64_t)Np * Np) * 2 < (1ll << 31) &&
      !(ep && ep[0] == '1');
  // 0. weights: the forward's packing and the transposed packs, batched
  //    into three launches
  Carve pc(a.packed, SIZE_MAX);
  TriMulPacked<T> w = carve_trimul<T>(pc, CZ, CH);
  {
    PackScope batch(st);
    if ((rc = gtk_tri_mul_pack(wts, CZ, CH, dtype, a.packed, gtk_tri_mul_packed_size(CZ, CH, dtype), st)))
      return rc;
    if ((rc = launch_pack_acc<T>(a.wzt, wts->z_w, wd, CH, CZ, 1, CH, st))) return rc;
    const void* wsrc[4] = {wts->a_p_w, wts->a_g_w, wts->b_p_w, wts->b_g_w};
    for (int k = 0; k < 4; ++k)
      if ((rc = launch_pack_acc<T>(a.wt + k * packed_elems(CZ, CH), wsrc[k], wd, CZ, CH, 1, CZ, st)))
        return rc;
    if ((rc = launch_pack_acc<T>(a.wgt, wts->g_w, wd, CZ, CZ, 1, CZ, st))) return rc;
    if ((rc = batch.flush())) return rc;
  }
  // 1. forward planes
  if ((rc = trimul_recompute_planes(z, mask, a.packed, B, N, CZ, CH, outgoing, eps_in, dtype, a.pa,
                                    a.pb, a.px, st)))
    return rc;
  // 2. epilogue backward
  {
    const int64_t tiles = B * (int64_t)Np * (Np / 32);
    StageTimer timer("trimul_bwd_epilogue", st);
    auto epi = [&](auto full, auto stg) {
      trimul_bwd_epilogue_kernel<T, CZ, CH, decltype(full)::value, decltype(stg)::value>
          <<<(unsigned)((tiles + 3) / 4), 256, 0, st>>>(
              (const T*)z, a.px, (const T*)dy, a.pdx, a.cm_dp, a.cm_stack + (int64_t)4 * CH * pitch,
              a.cm_xo, a.cm_dxo, w, a.wzt, (int)B, (int)N, Np, pitch, eps_in, eps_out);
    };
    using BF = std::integral_constant<bool, sizeof(T) == 2>;
    bool lds = false;
    if constexpr (sizeof(T) == 2 && trimul_folded<CZ, CH>()) {
      if (fits32 && N % 32 == 0) {
        const int grid = (int)std::min<int64_t>(device_cus(), (tiles + 3) / 4);
        trimul_bwd_epilogue_lds_kernel<CZ, CH><<<grid, 256, 0, st>>>(
            (const bf16*)z, a.px, (const bf16*)dy, a.pdx, a.cm_dp, a.cm_stack + (int64_t)4 * CH * pitch, a.cm_xo,
            a.cm_dxo, w, a.wzt, (int)B, (int)N, Np, pitch, eps_in, eps_out, tiles);
        lds = true;
      }
    }
    if (lds) {
    } else if (!fits32) {
      epi(std::false_type{}, std::false_type{});
    } else if (sizeof(T) == 2 && N % 32 == 0) {
      epi(BF{}, std::true_type{});
    } else {
      epi(std::false_type{}, std::true_type{});
    }
    GTK_LAUNCH_CHECK();
  }
  // 3. contraction backward.  Outgoing: dA = dX Bm, dB = dX^T A; incoming
  // (planes stored so that X = A Bm^T as well): dA^T = Bm^T dX, dB^T =
  // A^T dX^T.  The bf16 tile kernels read the operands that enter
  // transposed straight from the planes (trimul_contract_planes_t);
  // otherwise the planes are transposed first (px is free from here on: it
  // takes dX^T).  GENIE_TK_TRANSPOSE_PLANES=1 selects the transposing form
  // everywhere (for tests: the two forms give identical bits).
  if (!a.pat) {
    if (outgoing) {
      if ((rc = trimul_contract_planes_t(a.pdx, a.pb, a.pda, Np, nplanes, false, true, st))) return rc;
      if ((rc = trimul_contract_planes_t(a.pdx, a.pa, a.pdb, Np, nplanes, true, true, st))) return rc;
    } else {
      if ((rc = trimul_contract_planes_t(a.pb, a.pdx, a.pda, Np, nplanes, true, false, st))) return rc;
      if ((rc = trimul_contract_planes_t(a.pa, a.pdx, a.pdb, Np, nplanes, true, true, st))) return rc;
    }
  } else {
    T* pdxt = a.px;
    if ((rc = launch_transpose_planes<T>(a.pa, a.pat, Np, nplanes, st))) return rc;
    if ((rc = launch_transpose_planes<T>(a.pb, a.pbt, Np, nplanes, st))) return rc;
    if ((rc = launch_transpose_planes<T>(a.pdx, pdxt, Np, nplanes, st))) return rc;
    if (outgoing) {
      if ((rc = trimul_contract_planes(a.pdx, a.pbt, a.pda, Np, nplanes, dtype, st))) return rc;
      if ((rc = trimul_contract_planes(pdxt, a.pat, a.pdb, Np, nplanes, dtype, st))) return rc;
    } else {
      if ((rc = trimul_contract_planes(a.pbt, a.pdx, a.pda, Np, nplanes, dtype, st))) return rc;
      if ((rc = trimul_contract_planes(a.pat, pdxt, a.pdb, Np, nplanes, dtype, st))) return rc;
    }
  }
  // 4. prologue backward
  {
    const int64_t tiles = B * N * ((N + 31) / 32);
    StageTimer timer("trimul_bwd_prologue", st);
    bool sides = false;
    if constexpr (sizeof(T) == 2) {
      if (fits32) {
        const int grid = (int)std::min<int64_t>(device_cus(), (tiles + 7) / 8);
        auto side = [&](auto full) -> int {
          constexpr bool F = decltype(full)::value;
          trimul_bwd_prologue_side_kernel<CZ, CH, 0, F><<<grid, 512, 0, st>>>(
              (const bf16*)z, mask, a.pda, (bf16*)dz, a.cm_stack, a.cm_xi, a.cm_dzn, w, a.wt, a.wgt,
              a.part_dzn, (int)B, (int)N, Np, pitch, eps_in, tiles);
          GTK_LAUNCH_CHECK();
          trimul_bwd_prologue_side_kernel<CZ, CH, 1, F><<<grid, 512, 0, st>>>(
              (const bf16*)z, mask, a.pdb, (bf16*)dz, a.cm_stack, a.cm_xi, a.cm_dzn, w, a.wt, a.wgt,
              a.part_dzn, (int)B, (int)N, Np, pitch, eps_in, tiles);
          GTK_LAUNCH_CHECK();
          return 0;
        };
        // whole 32-pair tiles on one row: the staged channel-major path
        if ((rc = N % 32 == 0 ? side(std::true_type{}) : side(std::false_type{}))) return rc;
        sides = true;
      }
    }
    if (!sides)
      trimul_bwd_prologue_kernel<T, CZ, CH><<<(unsigned)((tiles + 3) / 4), 256, 0, st>>>(
          (const T*)z, mask, a.pda, a.pdb, (T*)dz, a.cm_stack, a.cm_xi, a.cm_dzn, w, a.wt, a.wgt,
          (int)B, (int)N, Np, pitch, eps_in);
    GTK_LAUNCH_CHECK();
  }
  // 5. weight gradients
  if ((rc = launch_zero_tail<T>(a.cm_stack, M1, pitch, P, st))) return rc;
  if ((rc = launch_zero_tail<T>(a.cm_dp, CZ, pitch, P, st))) return rc;
  if ((rc = launch_zero_tail<T>(a.cm_xi, CZ, pitch, P, st))) return rc;
  if ((rc = launch_zero_tail<T>(a.cm_xo, CH, pitch, P, st))) return rc;
  // LayerNorm parameter gradients straight into the outputs where requested
  auto or_tmp = [](float* dst, float* tmp) { return dst ? dst : tmp; };
  if ((rc = launch_rowred<T>(a.cm_dzn, a.cm_xi, CZ, pitch, P, a.red, or_tmp(gr->ln_in_b, a.sums_dzn),
                             or_tmp(gr->ln_in_w, a.dots_dzn), st)))
    return rc;
  if ((rc = launch_rowred<T>(a.cm_dxo, a.cm_xo, CH, pitch, P, a.red, or_tmp(gr->ln_out_b, a.sums_dxo),
                             or_tmp(gr->ln_out_w, a.dots_dxo), st)))
    return rc;
  // the weight-gradient products also sum their G rows: the bias gradients
  float* const sums_dp = or_tmp(gr->z_b, a.sums_dp);
  {
    StageTimer timer("trimul_bwd_wgrad", st);
    if ((rc = launch_wgrad<T>(a.cm_stack, a.cm_xi, a.part1, M1, CZ, pitch, st, a.rs, a.sums_stack))) return rc;
    if ((rc = launch_wgrad<T>(a.cm_dp, a.cm_xo, a.part2, CZ, CH, pitch, st, a.rs, sums_dp))) return rc;
  }
  float* wdst[5] = {gr->a_p_w, gr->a_g_w, gr->b_p_w, gr->b_g_w, gr->g_w};
  float* bdst[5] = {gr->a_p_b, gr->a_g_b, gr->b_p_b, gr->b_g_b, gr->g_b};
  CopyList biases;
  WgradSegs wsegs;
  for (int k = 0; k < 5; ++k) {
    const int m0 = k * CH, rows = k < 4 ? CH : CZ;
    wsegs.add(wdst[k], m0, rows);
    biases.add(bdst[k], a.sums_stack + m0, rows);
  }
  if ((rc = launch_wgrad_finish(a.part1, M1, CZ, pitch, wsegs, a.sums_stack, w.ln_in_w, w.ln_in_b, st)))
    return rc;
  if ((rc = launch_copy_list(biases, st))) return rc;
  if ((rc = launch_wgrad_finish(a.part2, CZ, CH, pitch, 0, CZ, sums_dp, w.ln_out_w, w.ln_out_b,
                                gr->z_w, st)))
    return rc;
  return GTK_OK;
}

}  // namespace gtk

using namespace gtk;

// Shapes of the backward kernels: c_z and c in {32, 64, 128}.
static bool trimul_bwd_shape_ok(int64_t c_z, int64_t c) {
  return (c_z == 32 || c_z == 64 || c_z == 128) && (c == 32 || c == 64 || c == 128);
}

template <typename T, int CZ>
static int bwd_trimul_c(int64_t c, const void* z, const float* mask, const void* dy,
                        const gtk_tri_mul_weights* w, void* dz, const gtk_tri_mul_grads* grads,
                        int64_t B, int64_t N, int outgoing, float eps_in, float eps_out, int dtype,
                        void* ws, hipStream_t st) {
  switch (c) {
    case 32: return bwd_trimul<T, CZ, 32>(z, mask, dy, w, dz, grads, B, N, outgoing, eps_in, eps_out, dtype, ws, st);
    case 64: return bwd_trimul<T, CZ, 64>(z, mask, dy, w, dz, grads, B, N, outgoing, eps_in, eps_out, dtype, ws, st);
    default: return bwd_trimul<T, CZ, 128>(z, mask, dy, w, dz, grads, B, N, outgoing, eps_in, eps_out, dtype, ws, st);
  }
}

template <typename T>
static int bwd_trimul_any(int64_t c_z, int64_t c, const void* z, const float* mask, const void* dy,
                          const gtk_tri_mul_weights* w, void* dz, const gtk_tri_mul_grads* grads,
                          int64_t B, int64_t N, int outgoing, float eps_in, float eps_out, int dtype,
                          void* ws, hipStream_t st) {
  switch (c_z) {
    case 32: return bwd_trimul_c<T, 32>(c, z, mask, dy, w, dz, grads, B, N, outgoing, eps_in, eps_out, dtype, ws, st);
    case 64: return bwd_trimul_c<T, 64>(c, z, mask, dy, w, dz, grads, B, N, outgoing, eps_in, eps_out, dtype, ws, st);
    default: return bwd_trimul_c<T, 128>(c, z, mask, dy, w, dz, grads, B, N, outgoing, eps_in, eps_out, dtype, ws, st);
  }
}

extern "C" size_t gtk_tri_mul_backward_workspace_size(int64_t B, int64_t N, int64_t c_z, int64_t c,
                                                      int dtype) {
  if (!trimul_bwd_shape_ok(c_z, c) || B < 0 || N < 0) return 0;
  if (dtype != GTK_F32 && dtype != GTK_BF16) return 0;
  Carve cv(nullptr, SIZE_MAX);
  if (dtype == GTK_F32) carve_trimul_bwd<float>(cv, B, N, (int)c_z, (int)c, dtype);
  else carve_trimul_bwd<bf16>(cv, B, N, (int)c_z, (int)c, dtype);
  return cv.off;
}

extern "C" int gtk_tri_mul_backward(const void* z, const float* mask, const void* dy,
                                    const gtk_tri_mul_weights* w, void* dz,
                                    const gtk_tri_mul_grads* grads, int64_t B, int64_t N,
                                    int64_t c_z, int64_t c, int outgoing, float eps_in,
                                    float eps_out, int dtype, void* ws, size_t ws_bytes,
                                    void* stream) {
  GTK_REQUIRE(dtype == GTK_F32 || dtype == GTK_BF16, GTK_EINVAL, "gtk_tri_mul_backward: bad dtype %d", dtype);
  GTK_REQUIRE(trimul_bwd_shape_ok(c_z, c), GTK_EUNSUPPORTED,
              "gtk_tri_mul_backward: c_z=%lld c=%lld unsupported (c_z and c in {32, 64, 128})",
              (long long)c_z, (long long)c);
  GTK_REQUIRE(B >= 0 && N >= 0 && N <= 4096, GTK_EINVAL, "gtk_tri_mul_backward: bad shape");
  if (B == 0 || N == 0) return GTK_OK;
  GTK_REQUIRE(z && dy && w && dz && grads && ws, GTK_EINVAL, "gtk_tri_mul_backward: null pointer");
  GTK_REQUIRE(w->dtype == GTK_F32 || w->dtype == GTK_BF16, GTK_EINVAL,
              "gtk_tri_mul_backward: bad weight dtype %d", w->dtype);
  GTK_REQUIRE(w->a_p_w && w->a_g_w && w->b_p_w && w->b_g_w && w->g_w && w->z_w, GTK_EINVAL,
              "gtk_tri_mul_backward: null weight");
  const float* gp[] = {grads->ln_in_w, grads->ln_in_b, grads->a_p_w, grads->a_p_b, grads->a_g_w,
                       grads->a_g_b, grads->b_p_w, grads->b_p_b, grads->b_g_w, grads->b_g_b,
                       grads->g_w, grads->g_b, grads->ln_out_w, grads->ln_out_b, grads->z_w,
                       grads->z_b};
  for (const float* p : gp) GTK_REQUIRE(p, GTK_EINVAL, "gtk_tri_mul_backward: null gradient pointer");
  const size_t need = gtk_tri_mul_backward_workspace_size(B, N, c_z, c, dtype);
  GTK_REQUIRE(ws_bytes >= need, GTK_EWORKSPACE, "gtk_tri_mul_backward: workspace %zu < %zu bytes",
              ws_bytes, need);
  hipStream_t st = (hipStream_t)stream;
  if (dtype == GTK_F32)
    return bwd_trimul_any<float>(c_z, c, z, mask, dy, w, dz, grads, B, N, outgoing, eps_in, eps_out, dtype, ws, st);
  return bwd_trimul_any<bf16>(c_z, c, z, mask, dy, w, dz, grads, B, N, outgoing, eps_in, eps_out, dtype, ws, st);
}
