// PairTransition fused with the pair-stack residual and mask, for gfx950.
//
//   out = (p + W2 relu(W1 LN(p) + b1) + b2) * m        (residual and m optional)
//
// Reference: src/genie_tk/pair_transform.py:64-84 (PairTransition: LayerNorm ->
// Linear(c, n c) -> ReLU -> Linear(n c, c)) and :180-193 (PairTransformLayer:
// p = p + transition(p); p = p * mask).
//
// One wave owns 32 rows (pairs).  The row is normalised into MFMA fragments
// (the LayerNorm affine is folded into W1 and b1), then for every 32-unit
// hidden tile ht:
//   h   = W1[ht] . x                       8 MFMAs, accumulator lane = row,
//                                          registers = hidden units 8g+4h+r
//   hf  = bf16(relu(h + b1))               two B fragments, straight from the
//                                          accumulator registers
//   y  += W2[:, ht] . hf                   8 MFMAs
// W2 is packed in the hidden-unit order of those accumulator registers, so
// the 4c-wide hidden activation never leaves registers.  W1 and W2 (256 KiB
// at c = 128) stream through a 4-stage LDS ring, 16 KiB per hidden tile,
// shared by the 8 waves of a block; the block persists over row tiles.
//
// fp32 (and the backward's forward recompute) use a generic kernel of the
// same algebra: one wave per 32-row tile, weight fragments read from L2.
//
// Backward (gtk_pair_transition_backward), the gradients torch autograd
// gives the reference's PairTransition (pair_transform.py:79-84):
//   h = W1 xn + b1, a = relu(h), y = W2 a + b2, xn = x_hat * g + beta
//   da = W2^T dy, dh = da [h > 0], dxn = W1^T dh, dx = LN backward of dxn
//   dW2 = sum dy a^T, db2 = sum dy, dW1 = sum dh xn^T, db1 = sum dh,
//   dg = sum dxn x_hat, dbeta = sum dxn
// One kernel per 32-row tile recomputes h, forms da, dh, dxn and dx, and
// writes x_hat, dxn, dy, a and dh channel-major; the weight gradients are
// then split-K products and row sums over those planes (grad_util.hpp).
#include <algorithm>

#include "capi_util.hpp"
#include "common.hpp"
#include "grad_util.hpp"
#include "pack.hpp"

namespace gtk {

#ifndef PT_STAGES
#define PT_STAGES 4
#endif

// Packed parameters: W1 [hid][c] with the LayerNorm weight folded in
// (standard fragment order), b1' = b1 + W1 beta, W2 [c][hid] for contraction
// over the hidden units in the order the W1 accumulators produce them
// (launch_pack_acc: chunk 2*ht + gp, lane half h, element e <-> hidden unit
// ht*32 + 16*gp + 8*(e>>2) + 4*h + (e&3)), b2; ln_* are fp32 copies.
template <typename T> struct PtPackedT {
  T *w1, *w2;
  float *b1, *b2, *ln_w, *ln_b;
};
using PtPacked = PtPackedT<bf16>;

template <typename T>
static PtPackedT<T> carve_pt(Carve& cv, int c, int hid) {
  PtPackedT<T> p;
  p.w1 = cv.take<T>(packed_elems(hid, c));
  p.w2 = cv.take<T>(packed_elems(c, hid));
  p.b1 = cv.take<float>(hid);
  p.b2 = cv.take<float>(c);
  p.ln_w = cv.take<float>(c);
  p.ln_b = cv.take<float>(c);
  return p;
}

// s_waitcnt vmcnt(min(after, K) * RPW): the immediate must be a constant.
template <int RPW, int K>
__device__ __forceinline__ void wait_copies(int64_t after) {
  if constexpr (K == 0) {
    __builtin_amdgcn_s_waitcnt(0x0F70);
  } else {
    if (after >= K) __builtin_amdgcn_s_waitcnt(0x0F70 | (K * RPW));
    else wait_copies<RPW, K - 1>(after);
  }
}

template <int C, int HID>
__global__ __launch_bounds__(512) void pair_transition_bf16_kernel(
    const bf16* __restrict__ p, const float* __restrict__ mask, bf16* __restrict__ out, PtPacked w,
    int64_t rows, int residual, float eps, int64_t ntiles) {
  constexpr int WAVES = 8;
  constexpr int KC = C / 16;         // k chunks of the input
  constexpr int HT = HID / 32;       // hidden tiles
  constexpr int NT = C / 32;         // output tiles
  constexpr int W1T = KC * 512;      // W1 elements of one hidden tile
  constexpr int STAGE = W1T + NT * 2 * 512;  // + the W2 chunks of that hidden tile
  constexpr int REGIONS = KC + 2 * NT;       // 1 KiB copies per stage
  constexpr int RPW = REGIONS / WAVES;       // per wave
  constexpr int NS = PT_STAGES;
  static_assert(REGIONS % WAVES == 0 && HT >= NS && (NS & (NS - 1)) == 0 && (NS - 2) * RPW < 16,
                "stage split");
  __shared__ __attribute__((aligned(1024))) bf16 ring[NS][STAGE];
  __shared__ __attribute__((aligned(16))) float b1l[HID];
  __shared__ __attribute__((aligned(16))) float b2l[C];
  for (int t = threadIdx.x; t < HID; t += blockDim.x) b1l[t] = w.b1[t];
  for (int t = threadIdx.x; t < C; t += blockDim.x) b2l[t] = w.b2[t];

  const int lane = threadIdx.x & 63;
  const int wave = wave_id();
  const int half = lane >> 5;
  const int t32 = lane & 31;
  // The weight stream is the same for every row tile, so the ring runs on
  // across tiles: stage s holds hidden tile s % HT.  Region q < KC of a stage
  // is W1 chunk q of that hidden tile; region KC + 2*nt + gp is W2 chunk
  // 2*ht + gp of output tile nt.
  const int64_t first = (int64_t)blockIdx.x * WAVES;
  const int64_t stride = (int64_t)gridDim.x * WAVES;
  const int64_t iters = first < ntiles ? (ntiles - first + stride - 1) / stride : 0;
  const int64_t S = iters * HT;  // block-uniform: every wave runs the same barriers
  auto issue = [&](int64_t s) {
    bf16* dst = ring[s & (NS - 1)];
    const int ht = (int)(s % HT);
#pragma unroll
    for (int i = 0; i < RPW; ++i) {
      const int q = wave * RPW + i;
      const bf16* src;
      if (q < KC) {
        src = w.w1 + ((int64_t)ht * KC + q) * 512;
      } else {
        const int u = q - KC, nt = u >> 1, gp = u & 1;
        src = w.w2 + ((int64_t)nt * (HID / 16) + 2 * ht + gp) * 512;
      }
      g2lds16(src + lane * 8, dst + q * 512);
    }
  };
  // Stage s has landed once at most the copies of the stages issued after it
  // are outstanding: stages s+1 .. s+NS-2 (those that exist), RPW copies each.
  auto wait_stage = [&](int64_t s) { wait_copies<RPW, NS - 2>(S - 1 - s); };
  auto load_w1 = [&](Frag<bf16>* f1, int64_t s) {
    const bf16* sw1 = ring[s & (NS - 1)];
#pragma unroll
    for (int ks = 0; ks < KC; ++ks) load_wfrag_lds(f1[ks], sw1, 0, ks, KC);
  };
  __syncthreads();
  if (iters == 0) return;

  // Schedule of stage s (one hidden tile of one row tile):
  //   read its W2 fragments; h = W1 . x (W1 fragments read during stage s-1);
  //   wait for stage s+1, barrier, copy stage s+3 into the slot of stage s-1,
  //   read the W1 fragments of stage s+1; y += W2 . relu(h)
  // so the LDS reads of each half overlap the MFMAs of the other.
#pragma unroll
  for (int s0 = 0; s0 < NS - 1; ++s0)
    if (s0 < S) issue(s0);
  Frag<bf16> f1[KC];
  wait_stage(0);
  barrier_only();
  if (NS - 1 < S) issue(NS - 1);
  load_w1(f1, 0);
  // Row r of tile t: lane (t32, half) holds channels half*C/2 .. +C/2 of it.
  auto row_of = [&](int64_t it, int64_t& r) {
    const int64_t tile = first + it * stride + wave;  // waves past the last tile still stage and synchronise
    r = tile * 32 + t32;
    return tile < ntiles && r < rows;
  };
  // An invalid row reads row 0 instead: output row j depends on input row j
  // only, and the results of invalid rows are never stored.
  auto load_rows = [&](Frag<bf16>* raw, int64_t r) {
#pragma unroll
    for (int ch = 0; ch < KC; ++ch) raw[ch].load(p + r * C + half * (C / 2) + ch * 8);
  };
  Frag<bf16> raw[KC];
  {
    int64_t r0;
    const bool v0 = row_of(0, r0);
    load_rows(raw, v0 ? r0 : 0);
  }
  int64_t s = 0;
  for (int64_t it = 0; it < iters; ++it) {
    int64_t r;
    const bool valid = row_of(it, r);
    Frag<bf16> xf[KC];
    ln_frags_bf16<C>(xf, raw, eps);
    Frag<bf16> keep[KC];  // the input rows again, for the residual
#pragma unroll
    for (int ch = 0; ch < KC; ++ch) keep[ch] = raw[ch];
    f32x16 y[NT];
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) y[nt] = zero16();
#pragma unroll 1
    for (int ht = 0; ht < HT; ++ht, ++s) {
      const bf16* sw2 = ring[s & (NS - 1)] + W1T;
      Frag<bf16> f2[2 * NT];
#pragma unroll
      for (int q = 0; q < 2 * NT; ++q) load_wfrag_lds(f2[q], sw2, q >> 1, q & 1, 2);
      f32x16 h = mma0(f1[0], xf[0]);
#pragma unroll
      for (int ks = 1; ks < KC; ++ks) mma(h, f1[ks], xf[ks]);
      Frag<bf16> hf[2];
#pragma unroll
      for (int gp = 0; gp < 2; ++gp) {
        float v[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const int g = 2 * gp + (e >> 2), rr = e & 3;
          v[e] = fmaxf(h[4 * g + rr] + b1l[ht * 32 + 8 * g + 4 * half + rr], 0.f);
        }
        hf[gp].set(v);
        // computed here, before the barrier, not sunk below it
        asm volatile("" : "+v"(hf[gp].v));
      }
      if (s + 1 < S) {
        wait_stage(s + 1);
        barrier_only();  // stage s+1 visible to every wave; stage s fully read
        if (s + NS < S) issue(s + NS);
      }
      // after the last stage this reads a stale slot, unused
      load_w1(f1, s + 1);
#pragma unroll
      for (int nt = 0; nt < NT; ++nt)
#pragma unroll
        for (int gp = 0; gp < 2; ++gp) mma(y[nt], f2[2 * nt + gp], hf[gp]);
      // issue the W1 reads for stage s+1 ahead of these MFMAs
      __builtin_amdgcn_sched_group_barrier(0x100, KC, 0);      // LDS reads
      __builtin_amdgcn_sched_group_barrier(0x008, 2 * NT, 0);  // MFMAs
    }
    // Epilogue.  Every load (residual, mask, the next tile's rows) is issued
    // before the first store: vmcnt counts stores too, so a load issued after
    // a store cannot be waited for without waiting for that store as well.
    // The loads are unconditional (an invalid row reads row 0) so that the
    // epilogue is one straight-line block.
    const int64_t rc = valid ? r : 0;
    const bool res = residual && valid;
    const float m = mask ? mask[rc] : 1.f;
    {
      int64_t rn;
      const bool vn = row_of(it + 1, rn);  // past the last tile: invalid, reads row 0
      load_rows(raw, vn ? rn : 0);
    }
    // Residual in the accumulator layout: output group q (channels 8q + 4*half
    // + 0..3, q < 2*KC) sits in dwords 0-1 (q < KC) or 2-3 (q >= KC) of
    // keep[q mod KC] once dwords 2-3 of the lower half-wave are swapped with
    // dwords 0-1 of the upper one (v_permlane32_swap).
    bf16x4 pr[NT * 4];
#pragma unroll
    for (int ch = 0; ch < KC; ++ch) {
      typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
      u32x4 d = __builtin_bit_cast(u32x4, keep[ch].v);
      const auto s02 = __builtin_amdgcn_permlane32_swap(d[0], d[2], false, false);
      const auto s13 = __builtin_amdgcn_permlane32_swap(d[1], d[3], false, false);
      typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
      pr[ch] = __builtin_bit_cast(bf16x4, u32x2{s02[0], s13[0]});
      pr[ch + KC] = __builtin_bit_cast(bf16x4, u32x2{s02[1], s13[1]});
    }
    // Stores: the half-waves trade channel quads (v_permlane32_swap) so
    // that each lane writes two 16-byte pieces of 8 consecutive channels a
    // 32-channel block instead of four 8-byte ones; every lane takes part,
    // and the stores of rows past the end are dropped (out-of-range offset
    // of the tile's buffer descriptor).
    const int64_t tile = first + it * stride + wave;
    const auto ors = buf_rsrc_u(out + tile * 32 * C, (uint32_t)(32 * C * 2));
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
      uint32_t pk[4][2];
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int c0 = nt * 32 + 8 * g + 4 * half;
        const f32x4 b2 = *reinterpret_cast<const f32x4*>(b2l + c0);
        float o[4];
#pragma unroll
        for (int rr = 0; rr < 4; ++rr) {
          o[rr] = y[nt][4 * g + rr] + b2[rr];
          if (res) o[rr] += (float)pr[nt * 4 + g][rr];
          o[rr] *= m;
        }
        pk[g][0] = pack_bf16x2(o[0], o[1]);
        pk[g][1] = pack_bf16x2(o[2], o[3]);
      }
#pragma unroll
      for (int p2 = 0; p2 < 2; ++p2) {
        const auto s0 = __builtin_amdgcn_permlane32_swap(pk[2 * p2][0], pk[2 * p2 + 1][0], false, false);
        const auto s1 = __builtin_amdgcn_permlane32_swap(pk[2 * p2][1], pk[2 * p2 + 1][1], false, false);
        const uint4 c = half ? make_uint4(s0[0], s1[0], pk[2 * p2 + 1][0], pk[2 * p2 + 1][1])
                             : make_uint4(pk[2 * p2][0], pk[2 * p2][1], s0[1], s1[1]);
        const uint32_t off = (uint32_t)((t32 * C + nt * 32 + 16 * p2 + 8 * half) * 2);
        buf_store16(ors, valid ? off : kBufSkip, c);
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Generic forward (fp32; any T): one wave per 32-row tile, weights from L2.
//   h = W1 . x (accumulators: lane = row, registers = hidden units), relu +
//   b1 straight into two B fragments, y += W2 . relu(h) per hidden tile.
// ---------------------------------------------------------------------------
template <typename T, int C, int HID>
__global__ __launch_bounds__(256) void pair_transition_kernel(
    const T* __restrict__ p, const float* __restrict__ mask, T* __restrict__ out, PtPackedT<T> w,
    int64_t rows, int residual, float eps) {
  const int lane = threadIdx.x & 63;
  const int half = lane >> 5;
  const int t32 = lane & 31;
  const int64_t tile = (int64_t)blockIdx.x * 4 + wave_id();
  if (tile * 32 >= rows) return;
  const int64_t r = tile * 32 + t32;
  const bool valid = r < rows;
  const int64_t rr = valid ? r : 0;
  RowHalf<C> rh;
  load_row_half<T, C>(rh, p + rr * C, valid);
  const f32x2 st = row_stats<C>(rh, eps);
  Frag<T> xf[C / 16];
  ln_to_frags<T, C>(xf, rh, st);
  f32x16 y[C / 32];
#pragma unroll
  for (int nt = 0; nt < C / 32; ++nt) y[nt] = zero16();
#pragma unroll 1
  for (int ht = 0; ht < HID / 32; ++ht) {
    const f32x16 h = row_gemm_tile<T, C, true>(xf, w.w1, ht);
    float hv[16];
#pragma unroll
    for (int g = 0; g < 4; ++g)
#pragma unroll
      for (int q = 0; q < 4; ++q) hv[4 * g + q] = fmaxf(h[4 * g + q] + w.b1[ht * 32 + 8 * g + 4 * half + q], 0.f);
    Frag<T> hf[2];
    vals_to_frags<T>(hf, hv);
#pragma unroll
    for (int nt = 0; nt < C / 32; ++nt)
#pragma unroll
      for (int gp = 0; gp < 2; ++gp) {
        Frag<T> wf;
        load_wfrag<T>(wf, w.w2, nt, 2 * ht + gp, HID / 16);
        mma(y[nt], wf, hf[gp]);
      }
  }
  if (!valid) return;
  const float m = mask ? mask[rr] : 1.f;
#pragma unroll
  for (int nt = 0; nt < C / 32; ++nt)
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const int c0 = nt * 32 + 8 * g + 4 * half;
      const f32x4 xr = residual ? load4f(p + rr * C + c0) : f32x4{0.f, 0.f, 0.f, 0.f};
      float o[4];
#pragma unroll
      for (int q = 0; q < 4; ++q) o[q] = (y[nt][4 * g + q] + w.b2[c0 + q] + xr[q]) * m;
      store4(out + rr * C + c0, o[0], o[1], o[2], o[3]);
    }
}

// ---------------------------------------------------------------------------
// Backward, per 32-row tile (one wave): recompute x_hat and h, then per hidden
// tile da = W2^T dy (w2t: W2^T in standard fragment order), dh = da [h > 0],
// dxn += W1^T dh (w1t: W1^T, unfolded, for an operand from accumulators);
// then the LayerNorm backward dx = rstd (g dxn - mean(g dxn) - x_hat
// mean(g dxn x_hat)).  x_hat, dxn, dy (c rows) and a, dh (hid rows) go to
// channel-major planes of `pitch` columns for the weight gradients.
// ---------------------------------------------------------------------------
template <typename T, int C, int HID>
__global__ __launch_bounds__(256) void pair_transition_bwd_kernel(
    const T* __restrict__ p, const T* __restrict__ dy, T* __restrict__ dp, T* __restrict__ cm_xh,
    T* __restrict__ cm_dxn, T* __restrict__ cm_dy, T* __restrict__ cm_a, T* __restrict__ cm_dh,
    PtPackedT<T> w, const T* __restrict__ w2t, const T* __restrict__ w1t, int64_t rows,
    int64_t pitch, float eps) {
  const int lane = threadIdx.x & 63;
  const int half = lane >> 5;
  const int t32 = lane & 31;
  const int64_t tile = (int64_t)blockIdx.x * 4 + wave_id();
  if (tile * 32 >= rows) return;
  const int64_t r = tile * 32 + t32;
  const bool valid = r < rows;
  const int64_t rr = valid ? r : 0;
  RowHalf<C> rh;
  load_row_half<T, C>(rh, p + rr * C, valid);
  const f32x2 st = row_stats<C>(rh, eps);
  Frag<T> xf[C / 16];
  ln_to_frags<T, C>(xf, rh, st);
  Frag<T> dyf[C / 16];
  {
    RowHalf<C> dr;
    load_row_half<T, C>(dr, dy + rr * C, valid);
#pragma unroll
    for (int ch = 0; ch < C / 16; ++ch) dyf[ch].set(dr.v + 8 * ch);
  }
  f32x16 dxn[C / 32];
#pragma unroll
  for (int nt = 0; nt < C / 32; ++nt) dxn[nt] = zero16();
#pragma unroll 1
  for (int ht = 0; ht < HID / 32; ++ht) {
    const f32x16 h = row_gemm_tile<T, C, true>(xf, w.w1, ht);
    const f32x16 da = row_gemm_tile<T, C, true>(dyf, w2t, ht);
    float av[16], dhv[16];
#pragma unroll
    for (int g = 0; g < 4; ++g)
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const float hb = h[4 * g + q] + w.b1[ht * 32 + 8 * g + 4 * half + q];
        av[4 * g + q] = fmaxf(hb, 0.f);
        dhv[4 * g + q] = hb > 0.f ? da[4 * g + q] : 0.f;
      }
    if (valid) {
#pragma unroll
      for (int g = 0; g < 4; ++g)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const int64_t o = (int64_t)(ht * 32 + 8 * g + 4 * half + q) * pitch + rr;
          cm_a[o] = cvt<T>(av[4 * g + q]);
          cm_dh[o] = cvt<T>(dhv[4 * g + q]);
        }
    }
    Frag<T> dhf[2];
    vals_to_frags<T>(dhf, dhv);
#pragma unroll
    for (int nt = 0; nt < C / 32; ++nt)
#pragma unroll
      for (int gp = 0; gp < 2; ++gp) {
        Frag<T> wf;
        load_wfrag<T>(wf, w1t, nt, 2 * ht + gp, HID / 16);
        mma(dxn[nt], wf, dhf[gp]);
      }
  }
  // LayerNorm backward in the accumulator layout (lane = row, channels
  // nt*32 + 8g + 4*half + q); x_hat re-read in that layout
  float s1 = 0.f, s2 = 0.f;
#pragma unroll
  for (int nt = 0; nt < C / 32; ++nt)
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const int c0 = nt * 32 + 8 * g + 4 * half;
      const f32x4 xv = valid ? load4f(p + rr * C + c0) : f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const float xh = (xv[q] - st[0]) * st[1];
        const float dxh = w.ln_w[c0 + q] * dxn[nt][4 * g + q];
        s1 += dxh;
        s2 += dxh * xh;
      }
    }
  s1 += xor32(s1);
  s2 += xor32(s2);
  const float m1 = s1 * (1.0f / C), m2 = s2 * (1.0f / C);
  if (!valid) return;
#pragma unroll
  for (int nt = 0; nt < C / 32; ++nt)
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const int c0 = nt * 32 + 8 * g + 4 * half;
      const f32x4 xv = load4f(p + rr * C + c0);
      const f32x4 dv = load4f(dy + rr * C + c0);
      float o[4];
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const float xh = (xv[q] - st[0]) * st[1];
        const float dxh = w.ln_w[c0 + q] * dxn[nt][4 * g + q];
        o[q] = st[1] * (dxh - m1 - xh * m2);
        const int64_t cm = (int64_t)(c0 + q) * pitch + rr;
        cm_xh[cm] = cvt<T>(xh);
        cm_dxn[cm] = cvt<T>(dxn[nt][4 * g + q]);
        cm_dy[cm] = cvt<T>(dv[q]);
      }
      store4(dp + rr * C + c0, o[0], o[1], o[2], o[3]);
    }
}

// dst[n][m] = sum_s part[s][m][n]: a weight-gradient product finished into
// the transposed layout (dW2 [c][hid] from the product over hid x c).
static __global__ void wgrad_finish_t_kernel(const float* __restrict__ part, int nsplit, int M, int Nn,
                                             float* __restrict__ dst) {
  const int idx = blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= M * Nn) return;
  const int n = idx / M, m = idx % M;
  float acc = 0.f;
  for (int sp = 0; sp < nsplit; ++sp) acc += part[((int64_t)sp * M + m) * Nn + n];
  dst[idx] = acc;
}

static bool pt_shape_ok(int64_t c, int64_t n) { return (c == 128 || c == 64) && n == 4; }

template <typename T>
static int pack_pt(const gtk_pair_transition_weights* w, int ci, int hid, void* packed, hipStream_t st) {
  const int wd = w->dtype;
  PackScope batch(st);  // the packing launches issued as 3
  Carve cv(packed, SIZE_MAX);
  PtPackedT<T> p = carve_pt<T>(cv, ci, hid);
  int rc;
  if ((rc = launch_to_f32(p.ln_w, w->ln_w, wd, ci, 1.f, 1.f, st))) return rc;
  if ((rc = launch_to_f32(p.ln_b, w->ln_b, wd, ci, 1.f, 0.f, st))) return rc;
  if ((rc = launch_pack<T>(p.w1, w->w1, wd, hid, ci, ci, 1, 1.f, st, p.ln_w))) return rc;
  if ((rc = launch_fold_bias(p.b1, w->w1, w->b1, wd, p.ln_b, hid, ci, ci, 1, 1.f, st))) return rc;
  if ((rc = launch_pack_acc<T>(p.w2, w->w2, wd, ci, hid, hid, 1, st))) return rc;
  if ((rc = launch_to_f32(p.b2, w->b2, wd, ci, 1.f, 0.f, st))) return rc;
  return batch.flush();
}

template <typename T, int C, int HID>
static int launch_pt_generic(const void* p, const float* mask, void* out, const PtPackedT<T>& w,
                             int64_t rows, int residual, float eps, hipStream_t st) {
  const int64_t ntiles = (rows + 31) / 32;
  GTK_REQUIRE((ntiles + 3) / 4 < (1ll << 31), GTK_EUNSUPPORTED, "pair transition: too many rows");
  StageTimer timer("pair_transition", st);
  pair_transition_kernel<T, C, HID><<<(unsigned)((ntiles + 3) / 4), 256, 0, st>>>(
      (const T*)p, mask, (T*)out, w, rows, residual, eps);
  GTK_LAUNCH_CHECK();
  return GTK_OK;
}

// Backward workspace: the packed forward weights, W2^T and W1^T for the
// backward products, five channel-major planes, the split-K partials and the
// row sums.
template <typename T> struct PtBwdWs {
  void* packed;
  T *w2t, *w1t, *cm_xh, *cm_dxn, *cm_dy, *cm_a, *cm_dh;
  float *part1, *part2, *red, *rs, *sums_dh, *sums_dy, *sums_dxn, *dots_dxn;
  int64_t pitch;
};

template <typename T>
static PtBwdWs<T> carve_pt_bwd(Carve& cv, int64_t rows, int c, int hid) {
  PtBwdWs<T> a;
  a.pitch = round_up(rows, 64);
  Carve pc(nullptr, SIZE_MAX);
  carve_pt<T>(pc, c, hid);
  a.packed = cv.take<char>((int64_t)pc.off);
  a.w2t = cv.take<T>(packed_elems(hid, c));
  a.w1t = cv.take<T>(packed_elems(c, hid));
  a.cm_xh = cv.take<T>(c * a.pitch);
  a.cm_dxn = cv.take<T>(c * a.pitch);
  a.cm_dy = cv.take<T>(c * a.pitch);
  a.cm_a = cv.take<T>(hid * a.pitch);
  a.cm_dh = cv.take<T>(hid * a.pitch);
  a.part1 = cv.take<float>(wgrad_part_floats(hid, c, a.pitch));
  a.part2 = cv.take<float>(wgrad_part_floats(hid, c, a.pitch));
  a.red = cv.take<float>((int64_t)2 * hid * kRowSegs);
  a.rs = cv.take<float>(wgrad_rowsum_floats(hid, a.pitch));
  a.sums_dh = cv.take<float>(hid);
  a.sums_dy = cv.take<float>(c);
  a.sums_dxn = cv.take<float>(c);
  a.dots_dxn = cv.take<float>(c);
  return a;
}

template <typename T, int C, int HID>
static int bwd_pt(const void* p, const void* dy, const gtk_pair_transition_weights* wts, void* dp,
                  const gtk_pair_transition_grads* gr, int64_t rows, float eps, void* ws,
                  hipStream_t st) {
  Carve cv(ws, SIZE_MAX);
  PtBwdWs<T> a = carve_pt_bwd<T>(cv, rows, C, HID);
  const int64_t pitch = a.pitch;
  const int wd = wts->dtype;
  int rc;
  Carve pc(a.packed, SIZE_MAX);
  const PtPackedT<T> w = carve_pt<T>(pc, C, HID);
  {
    PackScope batch(st);  // the forward's packing and the transposed packs, batched
    if ((rc = pack_pt<T>(wts, C, HID, a.packed, st))) return rc;
    // W2^T as [hid][c] (element (u, o) = W2[o][u]); W1^T as [c][hid] for dh
    // taken from the accumulators
    if ((rc = launch_pack<T>(a.w2t, wts->w2, wd, HID, C, 1, HID, 1.f, st))) return rc;
    if ((rc = launch_pack_acc<T>(a.w1t, wts->w1, wd, C, HID, 1, C, st))) return rc;
    if ((rc = batch.flush())) return rc;
  }
  {
    const int64_t ntiles = (rows + 31) / 32;
    GTK_REQUIRE((ntiles + 3) / 4 < (1ll << 31), GTK_EUNSUPPORTED, "pair transition backward: too many rows");
    StageTimer timer("pair_transition_bwd", st);
    pair_transition_bwd_kernel<T, C, HID><<<(unsigned)((ntiles + 3) / 4), 256, 0, st>>>(
        (const T*)p, (const T*)dy, (T*)dp, a.cm_xh, a.cm_dxn, a.cm_dy, a.cm_a, a.cm_dh, w, a.w2t,
        a.w1t, rows, pitch, eps);
    GTK_LAUNCH_CHECK();
  }
  T* planes[5] = {a.cm_xh, a.cm_dxn, a.cm_dy, a.cm_a, a.cm_dh};
  const int prow[5] = {C, C, C, HID, HID};
  for (int k = 0; k < 5; ++k)
    if ((rc = launch_zero_tail<T>(planes[k], prow[k], pitch, rows, st))) return rc;
  // bias and LayerNorm gradients straight into the outputs where requested
  auto or_tmp = [](float* dst, float* tmp) { return dst ? dst : tmp; };
  if ((rc = launch_rowred<T>(a.cm_dy, nullptr, C, pitch, rows, a.red, or_tmp(gr->b2, a.sums_dy), nullptr, st)))
    return rc;
  if ((rc = launch_rowred<T>(a.cm_dxn, a.cm_xh, C, pitch, rows, a.red, or_tmp(gr->ln_b, a.sums_dxn),
                             or_tmp(gr->ln_w, a.dots_dxn), st)))
    return rc;
  {
    // the first product also sums its G rows (dh): the b1 gradient
    StageTimer timer("pair_transition_bwd_wgrad", st);
    if ((rc = launch_wgrad<T>(a.cm_dh, a.cm_xh, a.part1, HID, C, pitch, st, a.rs, a.sums_dh))) return rc;
    if ((rc = launch_wgrad<T>(a.cm_a, a.cm_dy, a.part2, HID, C, pitch, st))) return rc;
  }
  // dW1 = (sum dh x_hat^T) diag(g) + (sum dh) beta^T
  if ((rc = launch_wgrad_finish(a.part1, HID, C, pitch, 0, HID, a.sums_dh, w.ln_w, w.ln_b, gr->w1, st)))
    return rc;
  if (gr->w2) {
    wgrad_finish_t_kernel<<<(HID * C + 255) / 256, 256, 0, st>>>(a.part2, wgrad_plan(HID, pitch).nsplit,
                                                                 HID, C, gr->w2);
    GTK_LAUNCH_CHECK();
  }
  return launch_copy_f32(gr->b1, a.sums_dh, HID, st);
}

}  // namespace gtk

using namespace gtk;

extern "C" size_t gtk_pair_transition_packed_size(int64_t c, int64_t n, int dtype) {
  if ((dtype != GTK_BF16 && dtype != GTK_F32) || !pt_shape_ok(c, n)) return 0;
  Carve cv(nullptr, SIZE_MAX);
  if (dtype == GTK_BF16) carve_pt<bf16>(cv, (int)c, (int)(c * n));
  else carve_pt<float>(cv, (int)c, (int)(c * n));
  return cv.off;
}

extern "C" int gtk_pair_transition_pack(const gtk_pair_transition_weights* w, int64_t c, int64_t n,
                                        int dtype, void* packed, size_t packed_bytes,
                                        void* stream) {
  GTK_REQUIRE(w && packed, GTK_EINVAL, "gtk_pair_transition_pack: null pointer");
  GTK_REQUIRE(dtype == GTK_BF16 || dtype == GTK_F32, GTK_EINVAL, "gtk_pair_transition_pack: bad dtype %d",
              dtype);
  GTK_REQUIRE(w->dtype == GTK_F32 || w->dtype == GTK_BF16, GTK_EINVAL,
              "gtk_pair_transition_pack: bad weight dtype %d", w->dtype);
  GTK_REQUIRE(pt_shape_ok(c, n), GTK_EUNSUPPORTED,
              "gtk_pair_transition_pack: c=%lld n=%lld unsupported (c in {64,128}, n == 4)",
              (long long)c, (long long)n);
  GTK_REQUIRE(w->w1 && w->w2, GTK_EINVAL, "gtk_pair_transition_pack: null weight");
  const size_t need = gtk_pair_transition_packed_size(c, n, dtype);
  GTK_REQUIRE(packed_bytes >= need, GTK_EWORKSPACE, "gtk_pair_transition_pack: buffer %zu < %zu bytes",
              packed_bytes, need);
  hipStream_t st = (hipStream_t)stream;
  if (dtype == GTK_BF16) return pack_pt<bf16>(w, (int)c, (int)(c * n), packed, st);
  return pack_pt<float>(w, (int)c, (int)(c * n), packed, st);
}

extern "C" int gtk_pair_transition_forward(const void* p, const float* mask, void* out,
                                           const void* packed, int64_t rows, int64_t c, int64_t n,
                                           int residual, float eps, int dtype, void* stream) {
  GTK_REQUIRE(dtype == GTK_BF16 || dtype == GTK_F32, GTK_EINVAL,
              "gtk_pair_transition_forward: bad dtype %d", dtype);
  GTK_REQUIRE(pt_shape_ok(c, n), GTK_EUNSUPPORTED,
              "gtk_pair_transition_forward: c=%lld n=%lld unsupported (c in {64,128}, n == 4)",
              (long long)c, (long long)n);
  GTK_REQUIRE(rows >= 0 && rows <= ((int64_t)1 << 36), GTK_EINVAL,
              "gtk_pair_transition_forward: bad rows %lld", (long long)rows);
  if (rows == 0) return GTK_OK;
  GTK_REQUIRE(p && out && packed, GTK_EINVAL, "gtk_pair_transition_forward: null pointer");
  hipStream_t st = (hipStream_t)stream;
  Carve pc((void*)packed, SIZE_MAX);
  if (dtype == GTK_F32) {
    const PtPackedT<float> w = carve_pt<float>(pc, (int)c, (int)(c * n));
    if (c == 128) return launch_pt_generic<float, 128, 512>(p, mask, out, w, rows, residual, eps, st);
    return launch_pt_generic<float, 64, 256>(p, mask, out, w, rows, residual, eps, st);
  }
  const PtPacked w = carve_pt<bf16>(pc, (int)c, (int)(c * n));
  const int64_t ntiles = (rows + 31) / 32;
  const int grid = (int)std::min<int64_t>(device_cus(), (ntiles + 7) / 8);
  StageTimer timer("pair_transition", st);
  if (c == 128)
    pair_transition_bf16_kernel<128, 512><<<grid, 512, 0, st>>>(
        (const bf16*)p, mask, (bf16*)out, w, rows, residual, eps, ntiles);
  else
    pair_transition_bf16_kernel<64, 256><<<grid, 512, 0, st>>>(
        (const bf16*)p, mask, (bf16*)out, w, rows, residual, eps, ntiles);
  GTK_LAUNCH_CHECK();
  return GTK_OK;
}

extern "C" size_t gtk_pair_transition_backward_workspace_size(int64_t rows, int64_t c, int64_t n,
                                                              int dtype) {
  if ((dtype != GTK_BF16 && dtype != GTK_F32) || !pt_shape_ok(c, n) || rows < 0 ||
      rows > ((int64_t)1 << 31))
    return 0;
  Carve cv(nullptr, SIZE_MAX);
  if (dtype == GTK_BF16) carve_pt_bwd<bf16>(cv, rows, (int)c, (int)(c * n));
  else carve_pt_bwd<float>(cv, rows, (int)c, (int)(c * n));
  return cv.off;
}

extern "C" int gtk_pair_transition_backward(const void* p, const void* dy,
                                            const gtk_pair_transition_weights* w, void* dp,
                                            const gtk_pair_transition_grads* g, int64_t rows,
                                            int64_t c, int64_t n, float eps, int dtype, void* ws,
                                            size_t ws_bytes, void* stream) {
  GTK_REQUIRE(dtype == GTK_BF16 || dtype == GTK_F32, GTK_EINVAL,
              "gtk_pair_transition_backward: bad dtype %d", dtype);
  GTK_REQUIRE(pt_shape_ok(c, n), GTK_EUNSUPPORTED,
              "gtk_pair_transition_backward: c=%lld n=%lld unsupported (c in {64,128}, n == 4)",
              (long long)c, (long long)n);
  GTK_REQUIRE(rows >= 0 && rows <= ((int64_t)1 << 31), GTK_EINVAL,
              "gtk_pair_transition_backward: bad rows %lld", (long long)rows);
  GTK_REQUIRE(w && g, GTK_EINVAL, "gtk_pair_transition_backward: null weights or gradients");
  GTK_REQUIRE(w->dtype == GTK_F32 || w->dtype == GTK_BF16, GTK_EINVAL,
              "gtk_pair_transition_backward: bad weight dtype %d", w->dtype);
  if (rows == 0) return GTK_OK;
  GTK_REQUIRE(p && dy && dp && ws && w->w1 && w->w2 && w->b1 && w->b2 && w->ln_w && w->ln_b,
              GTK_EINVAL, "gtk_pair_transition_backward: null pointer");
  const size_t need = gtk_pair_transition_backward_workspace_size(rows, c, n, dtype);
  GTK_REQUIRE(ws_bytes >= need, GTK_EWORKSPACE, "gtk_pair_transition_backward: workspace %zu < %zu bytes",
              ws_bytes, need);
  hipStream_t st = (hipStream_t)stream;
  if (dtype == GTK_F32)
    return c == 128 ? bwd_pt<float, 128, 512>(p, dy, w, dp, g, rows, eps, ws, st)
                    : bwd_pt<float, 64, 256>(p, dy, w, dp, g, rows, eps, ws, st);
  return c == 128 ? bwd_pt<bf16, 128, 512>(p, dy, w, dp, g, rows, eps, ws, st)
                  : bwd_pt<bf16, 64, 256>(p, dy, w, dp, g, rows, eps, ws, st);
}
