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
#include <algorithm>

#include "capi_util.hpp"
#include "common.hpp"
#include "pack.hpp"

namespace gtk {

#ifndef PT_STAGES
#define PT_STAGES 4
#endif

// Packed parameters: W1 [hid][c] with the LayerNorm weight folded in
// (standard fragment order), b1' = b1 + W1 beta, W2 [c][hid] in accumulator
// order (pack_w2_kernel), b2; ln_* are fp32 copies used while packing.
struct PtPacked {
  bf16 *w1, *w2;
  float *b1, *b2, *ln_w, *ln_b;
};

static PtPacked carve_pt(Carve& cv, int c, int hid) {
  PtPacked p;
  p.w1 = cv.take<bf16>(packed_elems(hid, c));
  p.w2 = cv.take<bf16>(packed_elems(c, hid));
  p.b1 = cv.take<float>(hid);
  p.b2 = cv.take<float>(c);
  p.ln_w = cv.take<float>(c);
  p.ln_b = cv.take<float>(c);
  return p;
}

// W2 [c][hid] (nn.Linear layout) for contraction over the hidden units in the
// order the W1 accumulators produce them: chunk ks2 = 2*ht + gp, lane l
// (output row nt*32 + (l&31), half h = l>>5), element e <-> hidden unit
//   ht*32 + 16*gp + 8*(e>>2) + 4*h + (e&3).
template <typename Tin>
__global__ void pack_w2_kernel(bf16* __restrict__ dst, const Tin* __restrict__ src, int c_out,
                               int hid, int64_t total) {
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= total) return;
  const int kch = hid / 16;
  const int e = idx & 7;
  const int l = (idx >> 3) & 63;
  const int64_t rest = idx >> 9;
  const int ks2 = (int)(rest % kch);
  const int nt = (int)(rest / kch);
  const int ht = ks2 >> 1, gp = ks2 & 1, h = l >> 5;
  const int u = ht * 32 + 16 * gp + 8 * (e >> 2) + 4 * h + (e & 3);
  const int o = nt * 32 + (l & 31);
  dst[idx] = (bf16)(o < c_out ? to_f32(src[(int64_t)o * hid + u]) : 0.f);
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
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
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
    if (valid) {
#pragma unroll
      for (int nt = 0; nt < NT; ++nt)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const int c0 = nt * 32 + 8 * g + 4 * half;
          const f32x4 b2 = *reinterpret_cast<const f32x4*>(b2l + c0);
          float o[4];
#pragma unroll
          for (int rr = 0; rr < 4; ++rr) {
            o[rr] = y[nt][4 * g + rr] + b2[rr];
            if (res) o[rr] += (float)pr[nt * 4 + g][rr];
          }
          store4(out + r * C + c0, o[0] * m, o[1] * m, o[2] * m, o[3] * m);
        }
    }
  }
}

static bool pt_shape_ok(int64_t c, int64_t n) { return (c == 128 || c == 64) && n == 4; }

}  // namespace gtk

using namespace gtk;

extern "C" size_t gtk_pair_transition_packed_size(int64_t c, int64_t n, int dtype) {
  if (dtype != GTK_BF16 || !pt_shape_ok(c, n)) return 0;
  Carve cv(nullptr, SIZE_MAX);
  carve_pt(cv, (int)c, (int)(c * n));
  return cv.off;
}

extern "C" int gtk_pair_transition_pack(const gtk_pair_transition_weights* w, int64_t c, int64_t n,
                                        int dtype, void* packed, size_t packed_bytes,
                                        void* stream) {
  GTK_REQUIRE(w && packed, GTK_EINVAL, "gtk_pair_transition_pack: null pointer");
  GTK_REQUIRE(dtype == GTK_BF16, GTK_EUNSUPPORTED, "gtk_pair_transition_pack: bf16 only");
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
  const int ci = (int)c, hid = (int)(c * n), wd = w->dtype;
  Carve cv(packed, SIZE_MAX);
  PtPacked p = carve_pt(cv, ci, hid);
  int rc;
  if ((rc = launch_to_f32(p.ln_w, w->ln_w, wd, ci, 1.f, 1.f, st))) return rc;
  if ((rc = launch_to_f32(p.ln_b, w->ln_b, wd, ci, 1.f, 0.f, st))) return rc;
  if ((rc = launch_pack<bf16>(p.w1, w->w1, wd, hid, ci, ci, 1, 1.f, st, p.ln_w))) return rc;
  if ((rc = launch_fold_bias(p.b1, w->w1, w->b1, wd, p.ln_b, hid, ci, ci, 1, 1.f, st))) return rc;
  const int64_t total = packed_elems(ci, hid);
  const unsigned blocks = (unsigned)((total + 255) / 256);
  if (wd == GTK_F32)
    pack_w2_kernel<float><<<blocks, 256, 0, st>>>(p.w2, (const float*)w->w2, ci, hid, total);
  else
    pack_w2_kernel<bf16><<<blocks, 256, 0, st>>>(p.w2, (const bf16*)w->w2, ci, hid, total);
  GTK_LAUNCH_CHECK();
  return launch_to_f32(p.b2, w->b2, wd, ci, 1.f, 0.f, st);
}

extern "C" int gtk_pair_transition_forward(const void* p, const float* mask, void* out,
                                           const void* packed, int64_t rows, int64_t c, int64_t n,
                                           int residual, float eps, int dtype, void* stream) {
  GTK_REQUIRE(dtype == GTK_BF16, GTK_EUNSUPPORTED, "gtk_pair_transition_forward: bf16 only");
  GTK_REQUIRE(pt_shape_ok(c, n), GTK_EUNSUPPORTED,
              "gtk_pair_transition_forward: c=%lld n=%lld unsupported (c in {64,128}, n == 4)",
              (long long)c, (long long)n);
  GTK_REQUIRE(rows >= 0 && rows <= ((int64_t)1 << 36), GTK_EINVAL,
              "gtk_pair_transition_forward: bad rows %lld", (long long)rows);
  if (rows == 0) return GTK_OK;
  GTK_REQUIRE(p && out && packed, GTK_EINVAL, "gtk_pair_transition_forward: null pointer");
  hipStream_t st = (hipStream_t)stream;
  Carve pc((void*)packed, SIZE_MAX);
  const PtPacked w = carve_pt(pc, (int)c, (int)(c * n));
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
