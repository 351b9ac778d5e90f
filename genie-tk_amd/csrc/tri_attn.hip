// Triangle attention (starting / ending node) for gfx950.
//
// Both nodes run in "destination" coordinates: row r is the axis whose
// entries are independent attention problems, positions j inside a row are
// queries and keys.  Starting node: (r, j) = pair (i, j).  Ending node:
// (r, j) = pair (j, i) of the input, i.e. the transposed problem
// (ending(x, m) = starting(x^T, m^T)^T).
//
//  1. prologue: per pair, LN -> q (pre-scaled by log2(e)/sqrt(d)), k, v,
//     gate sigmoid(. + b_g) and the triangle bias (scaled by log2(e)), all on
//     the matrix cores.  Workspace layouts (Np = N rounded up to 128; all in
//     the compute type):
//        fp32 path and the raw op:
//          q, k  [B][Np r][H][Np j][32]     v^T [B][Np r][H][32][Np j]
//          gate  [B][Np r][Np j][c_h]       bias [B][H][Np q][Np k]
//        bf16 module path (channel-major, written as 32-byte runs):
//          q, k, v^T  [B][Np r][H][32][Np j]    gate [B][Np r][c_h][Np j]
//          bias       [B][H][Np q][Np k]
//  2. flash core: one wave = one head x 32 queries of one row; keys in tiles
//     of 32.  S^T = K Q^T is accumulated on top of the bias tile, so lane l
//     owns one query and 16 of its keys; the row max needs one lane^32
//     exchange.  Online softmax in fp32 with exp2, P cast to bf16 and
//     O^T += V^T P^T on the matrix cores.
//  3. fused epilogue (module forward): o * gate for all heads staged in LDS,
//     then the output projection W_o on the matrix cores, + b_o, optional
//     residual, stored back at the source pair.
//
// Masking: key k of row r is excluded when mask == 0.  A row without any
// valid key attends uniformly over all N keys: that is what the reference's
// additive -1e9 bias produces in fp32 (every logit rounds to -1e9).
#include <algorithm>
#include <type_traits>

#include "capi_util.hpp"
#include "common.hpp"
#include "pack.hpp"

namespace gtk {

constexpr int HD = 32;      // head dimension handled by the kernels
constexpr int MAXN = 8192;  // largest N of the attention entry points

// Packed parameters of one TriangleAttention.  The LayerNorm weight is folded
// into w_q/w_k/w_v/w_g/w_b and its bias into b_q/b_k/b_v/b_g/b_b (b = W beta
// + c); w_q and b_q also carry log2(e)/sqrt(d), w_b and b_b carry log2(e), so
// that the softmax runs on exp2; w_g and b_g carry -log2(e) (gate = 1 /
// (1 + 2^u)).  ln_* are fp32 copies used while packing.
// Every head is padded to HD = 32 channels (c_h -> H * HD): a head of d < 32
// channels gets zero weight rows in w_q/w_k/w_v/w_g (zero biases) and zero
// input columns in w_o, so its padded q, k and v channels are exactly zero
// (q.k and P V are unchanged) and its padded gate channels multiply zeros.
template <typename T> struct TriAttnPacked {
  T *w_q, *w_k, *w_v, *w_g, *w_b, *w_o;
  float *b_q, *b_k, *b_v, *b_g, *b_b, *b_o;
  float *ln_w, *ln_b;
};

template <typename T>
static TriAttnPacked<T> carve_triattn(Carve& cv, int cin, int /*ch*/, int H) {
  const int ch = H * HD;  // padded heads
  TriAttnPacked<T> p;
  p.w_q = cv.take<T>(packed_elems(ch, cin));
  p.w_k = cv.take<T>(packed_elems(ch, cin));
  p.w_v = cv.take<T>(packed_elems(ch, cin));
  p.w_g = cv.take<T>(packed_elems(ch, cin));
  p.w_b = cv.take<T>(packed_elems(H, cin));
  p.w_o = cv.take<T>(packed_elems(cin, ch));
  p.b_q = cv.take<float>(ch);
  p.b_k = cv.take<float>(ch);
  p.b_v = cv.take<float>(ch);
  p.b_g = cv.take<float>(ch);
  p.b_b = cv.take<float>(32);
  p.b_o = cv.take<float>(cin);
  p.ln_w = cv.take<float>(cin);
  p.ln_b = cv.take<float>(cin);
  return p;
}

template <typename T> struct AttnWs {
  T *q, *k, *vt, *gate, *bias;
  // (row, head) flash path (bf16 module forward with Np <= kFlashRhMaxNp),
  // else null: the gated attention output (B x rows x Np x c_h, fragment
  // order: see the flash kernel), and the
  // triangle bias without its per-head constant in bf16, B x H x Np x Np in
  // the flash kernel's fragment order (bias_frag_off; then bias is empty)
  T* og;
  bf16* biasfr;
  // (row, head) flash path, else null: the key-mask bits of every attention
  // row (B x Np x Np/32 words: bit j of word t is key 32t + j, set for a
  // mask value other than 1) and the flags of each key tile (B x Np x Np/32:
  // bit 0 some key below N without mask bias, bit 1 some mask value neither
  // 0 nor 1), written by the prologue's bias pass
  uint32_t* mbits;
  int* mflags;
  // q, k, v^T and the gate hold `rows` rows per batch element, from absolute
  // row r0 on: all Np rows from 0, or one chunk of rows (chunked attention).
  // The bias always holds every row.  (The fp32 and raw-op kernels use the
  // full layout only.)
  int64_t rows;
  int r0;
  __host__ __device__ int64_t row(int b, int r) const { return (int64_t)b * rows + (r - r0); }
};

// Rows and positions are padded to a multiple of the flash kernel's query block.
inline int64_t attn_pad(int64_t N) { return round_up(N, 128); }

// Largest padded N of the (row, head) flash path: K^T and V^T of one row and
// head (2 x 32 x Np bf16) stay in LDS.
constexpr int64_t kFlashRhMaxNp = 1024;

// Gated attention output og of the (row, head) path, in the output
// projection's B-fragment order: tile (workspace row, query tile qt) is 8
// chunks ks of [64 lanes][8 channels]; lane = 32 * (c >= c_h/2) + (q & 31)
// holds channels c = (c_h/2) * (lane >= 32) + 8 ks .. +7 of query q.  The
// projection kernel reads each chunk as 1 KiB contiguous.  Element offset of
// (og tile = workspace row * Np/32 + qt, chunk ks, lane):
__host__ __device__ __forceinline__ int64_t og_frag_off(int64_t tile, int ks, int lane) {
  return ((tile * 8 + ks) * 64 + lane) * 8;
}

// bf16 triangle bias of the (row, head) path, per batch element, in the
// flash kernel's S^T fragment order: tile (query tile qt, key tile kt) of
// head h is 2 slabs s of [64 lanes][8], lane = 32 * ((kk >> 2) & 1) + (q & 31)
// for the tile's key kk = 8g + 4 * ((kk >> 2) & 1) + rr (rr = kk & 3), at
// element 4 * (g & 1) + rr of slab s = g / 2: S^T register 4g + rr of the
// lane.  A wave loads its bias tile as 2 contiguous 1 KiB pieces.  Element
// offset of (h, query q, key tile kt, keys kk .. kk+3 with kk % 4 == 0):
__host__ __device__ __forceinline__ uint32_t bias_frag_off(int h, int q, int kt, int kk, int Np) {
  const int nt = Np / 32;
  const uint32_t tile = (uint32_t)((h * nt + (q >> 5)) * nt + kt);
  const int g = kk >> 3, hh = (kk >> 2) & 1;
  return ((tile * 2 + (g >> 1)) * 64 + hh * 32 + (q & 31)) * 8 + (g & 1) * 4;
}

// Position of key j inside a V^T row: within each group of 16 keys, keys
// 4..7 and 8..11 trade places, so that the 8 keys one lane feeds to the PV
// product (16c + 4h + {0..3} and 16c + 8 + 4h + {0..3}, h = lane half) are
// 8 consecutive elements at 16c + 8h.
__host__ __device__ __forceinline__ int vt_pos(int j) {
  return (j & ~15) | (j & 3) | ((j & 4) << 1) | ((j & 8) >> 1);
}

// rows = 0: every row (Np); otherwise a chunk of that many rows.  ch: the
// gate's channels (0: none, the raw op); fast: the bf16 module kernels
// (c_in = 128, H = 4), whose (row, head) flash path at Np <= kFlashRhMaxNp
// keeps the bias in fp32 fragment order and writes og.
template <typename T>
static AttnWs<T> carve_attn_ws(Carve& cv, int64_t B, int64_t Np, int H, int ch, int64_t rows = 0,
                               bool fast = true) {
  AttnWs<T> w;
  w.rows = rows > 0 ? rows : Np;
  w.r0 = 0;
  const int64_t qkv = B * w.rows * H * Np * HD;
  w.q = cv.take<T>(qkv);
  w.k = cv.take<T>(qkv);
  w.vt = cv.take<T>(qkv);
  w.gate = cv.take<T>(ch > 0 ? B * w.rows * Np * ch : 0);
  const bool rh = fast && ch > 0 && sizeof(T) == 2 && Np <= kFlashRhMaxNp;
  w.bias = rh ? nullptr : cv.take<T>(B * H * Np * Np);
  w.og = rh ? cv.take<T>(B * w.rows * Np * ch) : nullptr;
  w.biasfr = rh ? cv.take<bf16>(B * H * Np * Np) : nullptr;
  w.mbits = rh ? cv.take<uint32_t>(B * Np * (Np / 32)) : nullptr;
  w.mflags = rh ? cv.take<int>(B * Np * (Np / 32)) : nullptr;
  return w;
}

// ---------------------------------------------------------------------------
// 1. Prologue (fused module path).  Destination rows r0 .. r0 + nrows - 1;
//    mode bit 0: q, k, v^T and the gate (into the workspace rows of ws), bit
//    1: the triangle bias (every row of it is read by every row's attention,
//    so row chunks compute it over all rows first).
// ---------------------------------------------------------------------------
template <typename T, int CIN, int H>
__global__ __launch_bounds__(256) void triattn_prologue_kernel(const T* __restrict__ x,
                                                               TriAttnPacked<T> w, AttnWs<T> ws,
                                                               int B, int N, int Np, int starting,
                                                               float eps, int r0, int nrows, int mode) {
  constexpr int CH = H * HD;
  const int lane = threadIdx.x & 63;
  const int half = lane >> 5;
  const int t32 = lane & 31;
  const int vtiles = Np / 32;
  const int64_t tile = (int64_t)blockIdx.x * 4 + wave_id();
  if (tile >= (int64_t)B * nrows * vtiles) return;
  const int vt = (int)(tile % vtiles);
  const int r = r0 + (int)((tile / vtiles) % nrows);  // destination row
  const int b = (int)(tile / ((int64_t)vtiles * nrows));
  const int j = vt * 32 + t32;                // destination position
  const bool valid = r < N && j < N;
  const int p = starting ? r : j, q = starting ? j : r;  // source pair
  const int64_t pair = ((int64_t)b * N + (valid ? p : 0)) * N + (valid ? q : 0);

  RowHalf<CIN> rh;
  load_row_half<T, CIN>(rh, x + pair * CIN, valid);
  const f32x2 st = row_stats<CIN>(rh, eps);
  Frag<T> xf[CIN / 16];
  ln_to_frags<T, CIN>(xf, rh, st);
  const float keep = valid ? 1.f : 0.f;

  const int64_t rowbase = ws.row(b, r);  // (b, r) in the workspace rows
#pragma unroll 1
  for (int h = 0; h < ((mode & 1) ? H : 0); ++h) {
    // q, k: [b][r][h][j][d], lane holds d = 8g + 4*half + rr -> 4 consecutive d
    const f32x16 aq = row_gemm_tile<T, CIN, true>(xf, w.w_q, h);
    const f32x16 ak = row_gemm_tile<T, CIN, true>(xf, w.w_k, h);
    const f32x16 av = row_gemm_tile<T, CIN, true>(xf, w.w_v, h);
    T* qd = ws.q + ((rowbase * H + h) * Np + j) * HD;
    T* kd = ws.k + ((rowbase * H + h) * Np + j) * HD;
    T* vd = ws.vt + (rowbase * H + h) * HD * (int64_t)Np + vt_pos(j);
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const int d0 = 8 * g + 4 * half;
      const float* bq = w.b_q + h * HD + d0;
      const float* bk = w.b_k + h * HD + d0;
      const float* bv = w.b_v + h * HD + d0;
      store4(qd + d0, (aq[4 * g] + bq[0]) * keep, (aq[4 * g + 1] + bq[1]) * keep,
             (aq[4 * g + 2] + bq[2]) * keep, (aq[4 * g + 3] + bq[3]) * keep);
      store4(kd + d0, (ak[4 * g] + bk[0]) * keep, (ak[4 * g + 1] + bk[1]) * keep,
             (ak[4 * g + 2] + bk[2]) * keep, (ak[4 * g + 3] + bk[3]) * keep);
#pragma unroll
      for (int rr = 0; rr < 4; ++rr) vd[(int64_t)(d0 + rr) * Np] = cvt<T>((av[4 * g + rr] + bv[rr]) * keep);
    }
  }
  // gate: [b][r][j][CH]
  T* gd = ws.gate + (rowbase * Np + j) * CH;
#pragma unroll 1
  for (int nt = 0; nt < ((mode & 1) ? CH / 32 : 0); ++nt) {
    const f32x16 ag = row_gemm_tile<T, CIN, true>(xf, w.w_g, nt);
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const int c0 = nt * 32 + 8 * g + 4 * half;
      store4(gd + c0, gate_from_u(ag[4 * g] + w.b_g[c0]), gate_from_u(ag[4 * g + 1] + w.b_g[c0 + 1]),
             gate_from_u(ag[4 * g + 2] + w.b_g[c0 + 2]), gate_from_u(ag[4 * g + 3] + w.b_g[c0 + 3]));
    }
  }
  // triangle bias: [b][h][r][j] (rows h >= H of the packed tile are zero)
  if (mode & 2) {
    const f32x16 ab = row_gemm_tile<T, CIN, true>(xf, w.w_b, 0);
    if (half == 0) {
#pragma unroll
      for (int rr = 0; rr < 4; ++rr)
        if (rr < H) ws.bias[(((int64_t)b * H + rr) * Np + r) * Np + j] = cvt<T>((ab[rr] + w.b_b[rr]) * keep);
    }
    if (H > 4) {
#pragma unroll
      for (int g = 0; g < 4; ++g)
#pragma unroll
        for (int rr = 0; rr < 4; ++rr) {
          const int h = 8 * g + 4 * half + rr;
          if (h >= 4 && h < H) ws.bias[(((int64_t)b * H + h) * Np + r) * Np + j] = cvt<T>((ab[4 * g + rr] + w.b_b[h]) * keep);
        }
    }
  }
}

// ---------------------------------------------------------------------------
// 1b. bf16 prologue: persistent, one 1024-thread block per CU with the packed
//     q/k/v/gate weights and the triangle-bias tile resident in LDS
//     (4 x 32 KiB + 8 KiB, direct global->LDS copies) and the folded biases
//     beside them; each wave then loops over 32-pair tiles.
//     Lane i32 of a wave normalises pair 16*((i32>>2)&1) + 4*(i32>>3) + (i32&3)
//     of the tile and the pairs are the MFMA A operand, so every accumulator
//     lane holds 16 consecutive positions of one output channel.  All outputs
//     of this path are channel-major over positions (below): each lane writes
//     32 contiguous bytes, or, in the (row, head) path's tiles, its pieces
//     after a register swap so that each store writes 1 KiB whole.  Workspace
//     layouts of the bf16 path (Np = N rounded up to 128):
//        q, k  [B][Np r][H][32 d][Np j]    v^T [B][Np r][H][32 d][Np j] (vt_pos order)
//        gate  [B][Np r][c_h][Np j]        bias [B][H][Np q][Np k]
//     Padding values are those of triattn_prologue_kernel.
//     The (row, head) tiles leave as device-scope (sc1) buffer stores of
//     1 KiB runs (N = 256: 22.4 -> 20.0 us; no change at N = 512), and MODE
//     15 unrolls its 16 projection steps so that the wait for the next
//     tile's prefetched rows counts the stores behind them (73.5 -> 71.6 us
//     at N = 512).
// ---------------------------------------------------------------------------
// MODE bit 0: q, k, v^T and gate; bit 1: the triangle bias; bit 2: the bias
// in the flash kernel's fragment order without its per-head constant
// (ws.biasfr) instead of row-major (ws.bias); bit 3: q, k, v^T and gate in
// the tiled layout of the (row, head) flash kernel (each (row, head) block of
// 32 channels x Np positions as Np/32 tiles [32 channels][32 positions],
// 2 KiB contiguous) instead of channel-major rows.  The tiles cover rows r0
// .. r0 + nrows - 1 of every batch element: [B][nrows][Np / 32].
template <int CIN, int H, int MODE>
__global__ __launch_bounds__(1024) void triattn_prologue_bf16_kernel(
    const bf16* __restrict__ x, const float* __restrict__ mask, TriAttnPacked<bf16> w, AttnWs<bf16> ws,
    int N, int Np, int starting, float eps, int64_t ntiles, int r0, int nrows) {
  static_assert((MODE & 3) != 0 && MODE <= 15, "q/k/v/gate, bias, or both");
  constexpr int CH = H * HD;
  constexpr int KCH = CIN / 16;
  constexpr int PE = (CH / 32) * KCH * 512;  // one packed c_in -> c_h projection
  constexpr int PB = KCH * 512;              // the packed c_in -> H tile (rows >= H are zero)
  static_assert(CH / 32 == H, "one 32-channel tile per head");
  __shared__ __attribute__((aligned(1024))) bf16 wl[4 * PE + PB];
  __shared__ __attribute__((aligned(16))) float bl[4 * CH + 32];
  copy_to_lds_async(wl, w.w_q, PE * 2);
  copy_to_lds_async(wl + PE, w.w_k, PE * 2);
  copy_to_lds_async(wl + 2 * PE, w.w_v, PE * 2);
  copy_to_lds_async(wl + 3 * PE, w.w_g, PE * 2);
  copy_to_lds_async(wl + 4 * PE, w.w_b, PB * 2);
  for (int t = threadIdx.x; t < CH; t += blockDim.x) {
    bl[t] = w.b_q[t];
    bl[CH + t] = w.b_k[t];
    bl[2 * CH + t] = w.b_v[t];
    bl[3 * CH + t] = w.b_g[t];
  }
  if (threadIdx.x < 32) bl[4 * CH + threadIdx.x] = w.b_b[threadIdx.x];
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();

  const int lane = threadIdx.x & 63;
  const int half = lane >> 5;
  const int i32 = lane & 31;
  const int prow = 16 * ((i32 >> 2) & 1) + 4 * (i32 >> 3) + (i32 & 3);
  const int vtiles = Np / 32;
  // Tiles [B][Np rows r][vtiles], walked without divisions.  The input rows of
  // the next tile are loaded at the start of each tile, ahead of its stores:
  // loads complete in issue order, so waiting for rows loaded after a store
  // would wait for that store too.  A lane outside the pair grid reads pair 0
  // and normalises to zero.
  // tiles dealt round-robin over the blocks first, so a small problem still
  // reaches every CU (a block may then run fewer than 16 busy waves)
  const int64_t tstride = (int64_t)gridDim.x * 16;
  // wave-uniform (readfirstlane): the tile walk, row bases and buffer
  // resources then live in scalar registers
  const int wave = wave_id();
  int64_t tile = (int64_t)wave * gridDim.x + blockIdx.x;
  TileWalk tw;
  tw.init(tile, tstride, nrows, vtiles);  // row r0 + tw.r
  // (exists = false: a tile past the end, also read as pair 0).  With the
  // bias (mode bit 1) on the (row, head) path, also the mask value of key
  // position t.c * 32 + i32 of attention row r (pair (r, k) for the starting
  // node, (k, r) for the ending node; 1 outside the grid).
  constexpr bool kMaskBits = (MODE & 2) != 0;
  const bool mbits_on = kMaskBits && ws.mbits != nullptr;
  auto load_rows = [&](Frag<bf16>* raw, float& mv, const TileWalk& t, bool exists) {
    const int jo = t.c * 32 + prow;
    const int tr = r0 + t.r;
    const bool ok = exists && tr < N && jo < N;
    const int p = starting ? tr : jo, q = starting ? jo : tr;
    const bf16* src = x + (ok ? (((int64_t)t.b * N + p) * N + q) * CIN : 0) + half * (CIN / 2);
#pragma unroll
    for (int ch = 0; ch < KCH; ++ch) raw[ch].load(src + ch * 8);
    if (mbits_on) {
      const int k = t.c * 32 + i32;
      const bool mok = exists && mask != nullptr && tr < N && k < N;
      const int64_t mi = (int64_t)t.b * N * N + (starting ? (int64_t)tr * N + k : (int64_t)k * N + tr);
      mv = mok ? mask[mok ? mi : 0] : 1.f;
    }
  };
  Frag<bf16> raw[KCH];
  float mval = 1.f;  // the mask value of this tile's key position (mbits_on)
  // One tile.  Every path through it issues the same loads and stores (no
  // branch around any of them), and the first tile is peeled off the loop, so
  // the compiler's waits for the prefetched rows count the stores issued
  // after them instead of waiting for them.
  auto body = [&](const int64_t tile) {
    const int vt = tw.c;
    const int r = r0 + tw.r;  // destination row
    const int b = tw.b;
    const float m_this = mval;
    const int jown = vt * 32 + prow;            // this lane's pair (A/B operand side)
    Frag<bf16> xf[KCH];
    const bool valid = r < N && jown < N;
    ln_frags_bf16<CIN>(xf, raw, eps);
    if (!valid) {
#pragma unroll
      for (int ch = 0; ch < KCH; ++ch) xf[ch].zero();
    }
    {
      TileWalk nx = tw;
      nx.next();
      load_rows(raw, mval, nx, tile + tstride < ntiles);
    }
    const int64_t rowbase = ws.row(b, r);  // q/k/v^T/gate row in the workspace
    const int j0 = vt * 32 + 16 * half;         // first of this lane's 16 positions
    // validity of the 16 positions j0 + jj, as a bit mask
    const int nvalid = r < N ? min(max(N - j0, 0), 16) : 0;

    // q, k, v, gate: one 32-channel tile (one head) per step, one MFMA chain
    // each; lane (i32, half) ends with positions j0 .. j0+15 of channel i32
    auto step_body = [&](const int step) {
      const int kind = step / H;  // 0 q, 1 k, 2 v, 3 gate
      const int h = step % H;
      const bf16* wt = wl + kind * PE;
      Frag<bf16> fw;
      load_wfrag_lds(fw, wt, h, 0, KCH);
      f32x16 acc = mma0(xf[0], fw);
#pragma unroll
      for (int ks = 1; ks < KCH; ++ks) {
        load_wfrag_lds(fw, wt, h, ks, KCH);
        mma(acc, xf[ks], fw);
      }
      const float bc = bl[kind * CH + h * HD + i32];
      uint32_t pk[8];
      bf16* dst;
      if (kind == 3) {
        // gate = sigmoid, at every position (padding included)
#pragma unroll
        for (int m = 0; m < 16; m += 2)
          pk[m / 2] = pack_bf16x2(gate_from_u(acc[m] + bc), gate_from_u(acc[m + 1] + bc));
        dst = ws.gate + (rowbase * CH + h * HD + i32) * (int64_t)Np + j0;
        if constexpr ((MODE & 8) != 0) dst = ws.gate + (rowbase * CH + h * HD) * (int64_t)Np + vt * 1024;
      } else {
        // q, k, v: zero outside the N x N pair grid; v^T in vt_pos order, which
        // swaps bits 2 and 3 of the position inside its group of 16: packed
        // in position order, that exchanges words 2-3 with words 4-5 (a
        // select on the wave-uniform kind; permuting the accumulator index
        // instead made every element an indexed register move)
#pragma unroll
        for (int m = 0; m < 16; m += 2)
          pk[m / 2] = pack_bf16x2(m < nvalid ? acc[m] + bc : 0.f, m + 1 < nvalid ? acc[m + 1] + bc : 0.f);
        if (kind == 2) {
          const uint32_t w2 = pk[2], w3 = pk[3];
          pk[2] = pk[4];
          pk[3] = pk[5];
          pk[4] = w2;
          pk[5] = w3;
        }
        bf16* base = kind == 0 ? ws.q : kind == 1 ? ws.k : ws.vt;
        dst = base + ((rowbase * H + h) * HD + i32) * (int64_t)Np + j0;
        if constexpr ((MODE & 8) != 0) dst = base + (rowbase * H + h) * HD * (int64_t)Np + vt * 1024;
      }
      uint4* o = reinterpret_cast<uint4*>(dst);
      if constexpr ((MODE & 8) != 0) {
        // tile (2 KiB, 16-byte piece 4c + j for channel c, positions 8j ..
        // 8j+7): after v_permlane16_swap register set s holds channels 16s ..
        // 16s+15 (lane l: channel 16s + l%16, piece j = 2*(l/32) + (l/16)%2),
        // so that store s writes bytes 1024s .. 1024s+1023 whole (16-byte
        // pieces 32 bytes apart, as each lane holds them, wrote at 5.7 TB/s
        // against 6.5)
        uint32_t lo[4], hi[4];
#pragma unroll
        for (int d = 0; d < 4; ++d) {
          const auto sw = __builtin_amdgcn_permlane16_swap(pk[d], pk[4 + d], false, false);
          lo[d] = sw[0];
          hi[d] = sw[1];
        }
        const int sl = 4 * (lane & 15) + 2 * half + ((lane >> 4) & 1);
        const auto trs = buf_rsrc(dst, 2048);
        buf_store16_sc1(trs, (uint32_t)sl * 16, make_uint4(lo[0], lo[1], lo[2], lo[3]));
        buf_store16_sc1(trs, (uint32_t)(64 + sl) * 16, make_uint4(hi[0], hi[1], hi[2], hi[3]));
      } else {
        o[0] = make_uint4(pk[0], pk[1], pk[2], pk[3]);
        o[1] = make_uint4(pk[4], pk[5], pk[6], pk[7]);
      }
    };
    // MODE 15 unrolls the steps (a constant trip count, 128 VGPRs): the
    // compiler then counts the stores issued after the prefetched rows, so
    // the next tile's wait for them does not wait for this tile's stores.
    // The other modes would spill unrolled.
    if constexpr (MODE == 15) {
#pragma unroll
      for (int step = 0; step < 4 * H; ++step) step_body(step);
    } else {
#pragma unroll 1
      for (int step = 0; step < ((MODE & 1) ? 4 * H : 0); ++step) step_body(step);
    }
    // key-mask word and flags of (row r, key tile vt): bit j of the word is
    // key 32 vt + j (mask != 1); flags bit 0: some key below N without mask
    // bias, bit 1: some mask value neither 0 nor 1
    if (mbits_on) {
      const bool masked = m_this != 1.f;
      const uint32_t word = (uint32_t)__ballot(masked);  // lanes 0-31 (the upper half repeats them)
      const int nin = N - vt * 32;                         // keys of the tile below N
      const uint32_t inside = nin >= 32 ? 0xffffffffu : nin > 0 ? (1u << nin) - 1u : 0u;
      const int fl = ((inside & ~word) != 0u ? 1 : 0) |
                     (word != 0u && __ballot(masked && m_this != 0.f) != 0ull ? 2 : 0);
      const int64_t wi = ((int64_t)b * Np + r) * (Np / 32) + vt;
      if (lane == 0) {
        ws.mbits[wi] = word;
        ws.mflags[wi] = fl;
      }
    }
    // triangle bias [b][h][r][j]: lanes with i32 < H hold head i32
    if constexpr ((MODE & 2) != 0) {
      const bf16* wb = wl + 4 * PE + opaque_zero();
      Frag<bf16> fb;
      load_wfrag_lds(fb, wb, 0, 0, KCH);
      f32x16 ab = mma0(xf[0], fb);
#pragma unroll
      for (int ks = 1; ks < KCH; ++ks) {
        load_wfrag_lds(fb, wb, 0, ks, KCH);
        mma(ab, xf[ks], fb);
      }
      // lanes i32 >= H store nothing (out-of-range offset, no branch)
      const float bb = bl[4 * CH + (i32 & (H - 1))];
      if constexpr ((MODE & 4) != 0) {
        // bf16 in the flash kernel's S^T fragment order (bias_frag_off),
        // without the head's constant bb: a logit offset shared by every
        // query and key of the head, which the softmax cancels.  bb carries
        // the LayerNorm beta (folded in at packing), so what remains,
        // LN(x) . (gamma * w), is the part that varies between pairs.
        (void)bb;
        const auto brs = buf_rsrc(ws.biasfr + (int64_t)b * H * Np * Np, (uint32_t)(H * Np * Np * 2));
#pragma unroll
        for (int a = 0; a < 4; ++a) {
          // positions j0 + 4a .. +3: key kk = 16*half + 4a + rr of key tile vt
          const uint32_t off = i32 < H ? bias_frag_off(i32, r, vt, 16 * half + 4 * a, Np) * 2 : kBufSkip;
          float bv[4];
#pragma unroll
          for (int rr = 0; rr < 4; ++rr) bv[rr] = 4 * a + rr < nvalid ? ab[4 * a + rr] : 0.f;
          buf_store4(brs, off, bv[0], bv[1], bv[2], bv[3]);
        }
      } else {
        uint32_t pk[8];
#pragma unroll
        for (int m = 0; m < 16; m += 2)
          pk[m / 2] = pack_bf16x2(m < nvalid ? ab[m] + bb : 0.f, m + 1 < nvalid ? ab[m + 1] + bb : 0.f);
        const auto brs = buf_rsrc(ws.bias + (int64_t)b * H * Np * Np, (uint32_t)(H * Np * Np * 2));
        const uint32_t off = i32 < H ? (uint32_t)((((int64_t)i32 * Np + r) * Np + j0) * 2) : kBufSkip;
        buf_store16(brs, off, make_uint4(pk[0], pk[1], pk[2], pk[3]));
        buf_store16(brs, off + 16, make_uint4(pk[4], pk[5], pk[6], pk[7]));
      }
    }
  };
  if (tile < ntiles) {
    load_rows(raw, mval, tw, true);
    body(tile);
    tile += tstride;
    tw.next();
  }
  for (; tile < ntiles; tile += tstride, tw.next()) body(tile);
}

// ---------------------------------------------------------------------------
// 2. Flash core: returns the normalised O^T tile of one (row, head, 32 queries)
//    lane l: query q0 + (l&31), o[4g + rr] <-> d = 8g + 4*(l>>5) + rr
// ---------------------------------------------------------------------------
struct MaskView {
  const float* m;  // nullptr: all valid
  int64_t row_stride, key_stride;
  float inf;       // a key's logit takes inf * (mask - 1)
};

template <typename T>
__device__ __forceinline__ f32x16 flash_row_head(const T* __restrict__ qh, const T* __restrict__ kh,
                                                 const T* __restrict__ vth,
                                                 const T* __restrict__ biash, MaskView mv,
                                                 int q0, int N, int Np) {
  const int lane = threadIdx.x & 63;
  const int half = lane >> 5;
  const int t32 = lane & 31;

  Frag<T> qf[2];
#pragma unroll
  for (int m = 0; m < 2; ++m) qf[m].load(qh + (int64_t)(q0 + t32) * HD + m * 16 + half * 8);
  const T* brow = biash + (int64_t)(q0 + t32) * Np;

  f32x16 o = zero16();
  float m_run = -INFINITY, l_run = 0.f;
  const int ktiles = (N + 31) / 32;
  for (int kt = 0; kt < ktiles; ++kt) {
    const int k0 = kt * 32;
    f32x16 s;
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const f32x4 bv = load4f(brow + k0 + 8 * g + 4 * half);
#pragma unroll
      for (int rr = 0; rr < 4; ++rr) s[4 * g + rr] = bv[rr];
    }
#pragma unroll
    for (int m = 0; m < 2; ++m) {
      Frag<T> kf;
      kf.load(kh + (int64_t)(k0 + t32) * HD + m * 16 + half * 8);
      mma(s, kf, qf[m]);
    }
    // padded keys take no weight; a masked key (mask != 1) takes the
    // reference's additive bias inf * (mask - 1), here in log2 units.  A row
    // whose keys are all masked follows the reference's fp32 arithmetic
    // (uniform for inf = 1e9: every score rounds to one value).
    const bool tail = k0 + 32 > N;
    if (tail || mv.m) {
#pragma unroll
      for (int g = 0; g < 4; ++g)
#pragma unroll
        for (int rr = 0; rr < 4; ++rr) {
          const int k = k0 + 8 * g + 4 * half + rr;
          if (k >= N) {
            s[4 * g + rr] = -INFINITY;
          } else if (mv.m) {
            const float mval = mv.m[k * mv.key_stride];
            if (mval != 1.f) s[4 * g + rr] += (mv.inf * (mval - 1.f)) * kLog2e;
          }
        }
    }
    float mt = s[0];
#pragma unroll
    for (int e = 1; e < 16; ++e) mt = fmaxf(mt, s[e]);
    mt = fmaxf(mt, xor32(mt));
    const float m_new = fmaxf(m_run, mt);
    const float m_use = (m_new == -INFINITY) ? 0.f : m_new;
    const float alpha = exp2f(m_run - m_use);
    float ls = 0.f;
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      s[e] = exp2f(s[e] - m_use);
      ls += s[e];
    }
    l_run = l_run * alpha + ls;
    m_run = m_new;
#pragma unroll
    for (int e = 0; e < 16; ++e) o[e] *= alpha;
#pragma unroll
    for (int c = 0; c < 2; ++c) {
      Frag<T> pf, vf;
      float pv[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) pv[e] = s[8 * c + e];
      pf.set(pv);
      // V^T fragment: row d = t32; slots e<4 -> key 16c+4h+e, e>=4 -> key
      // 16c+8+4h+(e-4): 8 consecutive elements at 16c+8h (see vt_pos)
      vf.load(vth + (int64_t)t32 * Np + k0 + 16 * c + 8 * half);
      mma(o, vf, pf);
    }
  }
  const float l_tot = l_run + xor32(l_run);
  const float inv = 1.0f / l_tot;
#pragma unroll
  for (int e = 0; e < 16; ++e) o[e] *= inv;
  return o;
}

// ---------------------------------------------------------------------------
// 3a. Fused module kernel: all H heads of 32 queries of one row per block.
// ---------------------------------------------------------------------------
template <typename T, int CIN, int H>
__global__ __launch_bounds__(64 * H) void triattn_fused_kernel(const T* __restrict__ x,
                                                               const float* __restrict__ mask,
                                                               T* __restrict__ out,
                                                               TriAttnPacked<T> w, AttnWs<T> ws,
                                                               int B, int N, int Np, int starting,
                                                               int residual, float inf, int r0,
                                                               int nrows) {
  constexpr int CH = H * HD;
  constexpr int OPITCH = CH + 8;
  __shared__ __attribute__((aligned(16))) T os[32 * OPITCH];
  const int lane = threadIdx.x & 63;
  const int h = wave_id();
  const int half = lane >> 5;
  const int t32 = lane & 31;
  const int qtiles = (N + 31) / 32;
  const int qt = blockIdx.x % qtiles;
  const int r = r0 + (blockIdx.x / qtiles) % nrows;  // rows r0 .. r0 + nrows - 1
  const int b = blockIdx.x / (qtiles * nrows);
  const int q0 = qt * 32;

  const int64_t rowbase = ws.row(b, r);
  MaskView mv;
  if (mask) {
    // starting: key k of row r is pair (r, k); ending: pair (k, r)
    mv.m = mask + (int64_t)b * N * N + (starting ? (int64_t)r * N : r);
    mv.row_stride = 0;
    mv.key_stride = starting ? 1 : N;
  } else {
    mv.m = nullptr;
    mv.row_stride = mv.key_stride = 0;
  }
  mv.inf = inf;
  const f32x16 o = flash_row_head<T>(ws.q + (rowbase * H + h) * Np * HD,
                                     ws.k + (rowbase * H + h) * Np * HD,
                                     ws.vt + (rowbase * H + h) * HD * (int64_t)Np,
                                     ws.bias + ((int64_t)b * H + h) * Np * Np, mv, q0, N, Np);
  // gate and stage o*g in LDS as [query][CH]
  {
    const T* gr = ws.gate + (rowbase * Np + q0 + t32) * CH + h * HD;
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const int d0 = 8 * g + 4 * half;
      const f32x4 gv = load4f(gr + d0);
      store4(os + t32 * OPITCH + h * HD + d0, o[4 * g] * gv[0], o[4 * g + 1] * gv[1],
             o[4 * g + 2] * gv[2], o[4 * g + 3] * gv[3]);
    }
  }
  __syncthreads();
  Frag<T> of[CH / 16];
#pragma unroll
  for (int ks = 0; ks < CH / 16; ++ks) of[ks].load(os + t32 * OPITCH + half * (CH / 2) + ks * 8);
  const int q = q0 + t32;
  const bool qvalid = q < N;
  const int p0 = starting ? r : q, p1 = starting ? q : r;
  const int64_t pair = ((int64_t)b * N + (qvalid ? p0 : 0)) * N + (qvalid ? p1 : 0);
  for (int nt = h; nt < CIN / 32; nt += H) {
    const f32x16 acc = row_gemm_tile<T, CH, true>(of, w.w_o, nt);
    if (qvalid) {
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int c0 = nt * 32 + 8 * g + 4 * half;
        float v[4];
#pragma unroll
        for (int rr = 0; rr < 4; ++rr) v[rr] = acc[4 * g + rr] + w.b_o[c0 + rr];
        if (residual) {
          const f32x4 xr = load4f(x + pair * CIN + c0);
#pragma unroll
          for (int rr = 0; rr < 4; ++rr) v[rr] += xr[rr];
        }
        store4(out + pair * CIN + c0, v[0], v[1], v[2], v[3]);
      }
    }
  }
}

// ---------------------------------------------------------------------------
// 3c. bf16 module kernel: 1024 threads = H heads x 4 query tiles of 32, for a
//     block of 128 queries of one row.
//   * Key blocks of 64 keys (K rows and V^T columns of all heads, 32 KiB)
//     stream into a 3-stage LDS ring with direct global->LDS loads
//     (global_load_lds_dwordx4), issued two blocks ahead: no staging VGPRs,
//     one barrier per block.  Tiles are XOR-swizzled in 16-byte chunks so the
//     fragment reads are bank-conflict free.
//   * The triangle bias enters on the matrix cores: S^T += I . Bias^T with a
//     constant identity fragment, so the bias tile needs no VALU work; its
//     16-byte bf16 fragments for the next block are fetched as soon as the
//     current ones have been consumed.
//   * Online softmax with lazy rescaling: the reference max only moves when a
//     tile exceeds it by more than 8 (log2 units); exponentials stay <= 2^8
//     and the result is exact after the final division by l.
// ---------------------------------------------------------------------------
// l in [2^-60, 2^64], tested on the bits: positive floats order as unsigned
// integers; NaN, zero, negative values and infinity fall outside.  (The
// softmax code is built without NaN semantics, so a float compare would not
// be guaranteed to reject a NaN.)
__device__ __forceinline__ bool l_in_range(float l) {
  return __float_as_uint(l) - 0x21800000u <= 0x5F800000u - 0x21800000u;
}

__device__ __forceinline__ float lane_pair_max(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float lane_pair_sum(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}


template <int CIN, int H, int QT>
__global__ __launch_bounds__(64 * H * QT) __attribute__((amdgpu_waves_per_eu(4))) void triattn_flash_kernel(
    const bf16* __restrict__ x, const float* __restrict__ mask, bf16* __restrict__ out,
    TriAttnPacked<bf16> w, AttnWs<bf16> ws, int N, int Np, int starting, int residual, int r0,
    int nrows, float inf) {
  constexpr int CH = H * HD;
  constexpr int QB = 32 * QT;              // queries per block (QT query tiles per head)
  constexpr int NW = H * QT;               // waves
  constexpr int KB = 64;                   // keys per stage
  constexpr int NS = QT == 4 ? 3 : 2;      // LDS ring stages
  constexpr bool WO_LDS = QT == 4;         // W_o staged in LDS (else read from L2)
  constexpr int OP = CH + 8;               // gated-o row pitch in LDS (elements)
  constexpr int HEAD_BYTES = KB * HD * 2;  // K (or V^T) bytes of one head per stage: 4 KiB
  constexpr int STAGE_BYTES = 2 * H * HEAD_BYTES;
  constexpr int RPW = (STAGE_BYTES / 1024) / NW;  // 1 KiB copy regions per wave per stage
  constexpr float kRescale = 8.0f;         // lazy-rescale threshold (log2 units)
  static_assert(H == 4 && (QT == 4 || QT == 2), "4 heads; 64 or 128 queries per block");
  static_assert(QB * OP * 2 <= NS * STAGE_BYTES, "o staging must fit in the ring");
  __shared__ __attribute__((aligned(1024))) char ring[NS][STAGE_BYTES];
  __shared__ __attribute__((aligned(1024))) bf16 wo_l[WO_LDS ? (CIN / 32) * (CH / 16) * 512 : 8];
  // keys of this row, one bit per key: bit j of word t is key 32t + j
  __shared__ unsigned kmask[MAXN / 32];  // mask != 1: takes the bias inf * (mask - 1)
  __shared__ unsigned kfrac[MAXN / 32];  // ... with mask != 0 (bias from the value)
  __shared__ unsigned kpad[MAXN / 32];   // key >= N: no weight
  __shared__ int row_dirty;  // some key of the row is masked or padding

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // uniform: scalar addressing
  const int half = lane >> 5;
  const int t32 = lane & 31;
  const int h = wave / QT;
  const int qt = wave % QT;
  const int qblocks = (N + QB - 1) / QB;
  // XCD-aware order: the query blocks of one row run back to back on one XCD
  const int64_t lin = xcd_remap(blockIdx.x, gridDim.x);
  // blocks cover rows r0 .. r0 + nrows - 1 of every batch element
  const int qb = (int)(lin % qblocks);
  const int r = r0 + (int)((lin / qblocks) % nrows);
  const int b = (int)(lin / ((int64_t)qblocks * nrows));
  const int q0 = qb * QB + qt * 32;
  const int64_t rowbase = ws.row(b, r);  // q/k/v^T/gate row in the workspace

  // mask of this row: key k is pair (r, k) (starting) or (k, r) (ending)
  const float* mrow = mask ? mask + (int64_t)b * N * N + (starting ? (int64_t)r * N : r) : nullptr;
  const int64_t mks = starting ? 1 : N;
  if (tid == 0) row_dirty = 0;
  __syncthreads();
  {
    bool dirty = false;
    for (int k0 = wave * 64; k0 < Np; k0 += NW * 64) {
      const int k = k0 + lane;
      const bool inrow = k < N;
      const float mval = inrow && mrow ? mrow[k * mks] : 1.f;
      const bool masked = mval != 1.f;
      dirty = dirty || masked || !inrow;
      const unsigned long long mb = __ballot(masked);
      const unsigned long long fb = __ballot(masked && mval != 0.f);
      const unsigned long long pb = __ballot(!inrow);
      if (lane == 0) {
        kmask[k0 / 32] = (unsigned)mb;
        kmask[k0 / 32 + 1] = (unsigned)(mb >> 32);
        kfrac[k0 / 32] = (unsigned)fb;
        kfrac[k0 / 32 + 1] = (unsigned)(fb >> 32);
        kpad[k0 / 32] = (unsigned)pb;
        kpad[k0 / 32 + 1] = (unsigned)(pb >> 32);
      }
    }
    if (__ballot(dirty) != 0ull && lane == 0) row_dirty = 1;
  }
  __syncthreads();
  // block-uniform flag, kept in a scalar register
  const bool row_clean = __builtin_amdgcn_readfirstlane(row_dirty) == 0;
  const float madd0 = -inf * kLog2e;  // the bias of a key with mask == 0 (log2 units)

  // Async stage load.  A stage holds, for each head, the K^T and the V^T
  // block of 64 keys ([32 d][64 keys] each, 4 KiB); each splits into two 2 KiB
  // sub-blocks of 32 keys (sb), rows d of 64 bytes.  A stage is 32 regions of
  // 1 KiB (64 lanes x 16 B): region r is kind r>>4 (K^T, V^T), head (r>>2)&3,
  // sub-block (r>>1)&1, rows 16*(r&1) .. +15; lane l lands at row l/4,
  // physical 16-byte chunk l%4.  K^T chunks are unswizzled: the transposing
  // reads of a 16-lane group cover 4 consecutive rows x 32 bytes and the
  // paired group the other halves, every bank once.  V^T chunk p of row d sits
  // at physical chunk p ^ ((d>>2)&3), so the 16-byte reads of rows d, d+4,
  // d+8, d+12 fall in distinct banks.  Wave w moves regions RPW*w ..
  // RPW*w + RPW-1, all of one kind.
  static_assert(2 * H * 4 == 32 && (16 % RPW) == 0, "32 regions per stage, one kind per wave");
  const int rg0 = wave * RPW;
  const bool k_region = rg0 < 16;  // the first half of the waves move K^T
  const bf16* gbase = (k_region ? ws.k : ws.vt) + (rowbase * H) * (int64_t)HD * Np;
  const uint32_t ring_lds = lds_addr(&ring[0][0]);
  auto issue_stage = [&](int stage, int k0) {
    // The per-lane offset is recomputed from the lane id here rather than
    // kept across the tile loop: at the register cap it would be spilled, and
    // a reload from scratch waits for every outstanding load.  It is the same
    // for every region; the rest of each source address is uniform.
    const uint32_t ln = (uint32_t)(lane + opaque_zero());
    const uint32_t p = k_region ? (ln & 3) : ((ln & 3) ^ ((ln >> 4) & 3));
    const uint32_t voff = ((ln >> 2) * (uint32_t)Np + 8 * p) * 2;
#pragma unroll
    for (int i = 0; i < RPW; ++i) {
      const int r = rg0 + i;
      const bf16* src = gbase + (int64_t)(((r >> 2) & 3) * HD + 16 * (r & 1)) * Np + 32 * ((r >> 1) & 1) + k0;
      g2lds16_sv(src, voff, ring_lds + stage * STAGE_BYTES + r * 1024);
    }
  };

  // W_o for the epilogue, fetched now so that it is not waited for at the end
  if constexpr (WO_LDS) copy_to_lds_async(wo_l, w.w_o, (int)sizeof(wo_l));
  // q and the gate are channel-major ([32 channels][Np positions] per row and
  // head); this wave's [32 channels][32 queries] tile of either goes through
  // LDS (a 2 KiB region per wave, 64-byte rows) and is read back transposed.
  // Copy j (0, 1) moves channels 16j .. 16j+15: lane l takes channel
  // 16j + l/4, queries 8*(l%4) .. +7.
  const bf16* q_src = ws.q + ((rowbase * H + h) * HD) * (int64_t)Np + q0;
  const bf16* g_src = ws.gate + (rowbase * CH + h * HD) * (int64_t)Np + q0;
  auto issue_cq = [&](const bf16* src, int stage) {
    const uint32_t ln = (uint32_t)(lane + opaque_zero());
    const uint32_t voff = ((ln >> 2) * (uint32_t)Np + (ln & 3) * 8) * 2;
#pragma unroll
    for (int j = 0; j < 2; ++j)
      g2lds16_sv(src + (int64_t)j * 16 * Np, voff, ring_lds + stage * STAGE_BYTES + wave * 2048 + j * 1024);
  };
  // Channels c0 .. c0+3 of this lane's query t32 (ds_read_b64_tr_b16: lane
  // (group G = lane/16, i = lane%16) reads channel c0 + i/4 at queries
  // 16*(G&1) + 4*(i%4) .. +3; c0 carries the lane's half)
  auto read_cq4 = [&](int stage, int c0) {
    const int i = lane & 15;
    return lds_read_tr16(ring[stage] + wave * 2048 + (c0 + (i >> 2)) * 64 +
                         (16 * ((lane >> 4) & 1) + 4 * (i & 3)) * 2);
  };
  // query fragments (filled once the q tile is in LDS)
  Frag<bf16> qf[2];
  // K fragments come from the K^T tile with transposing reads: fetching lane
  // (group G = lane/16, i = lane%16) reads d row (i/4) of a 4-row group at
  // keys 16*(G&1) + 4*(i%4) .. +3 of the 32-key tile; the receiving lane
  // (key t32, half) gets d .. d+3 of its key
  const int trG = lane >> 4;
  const int tr_m = (lane & 15) >> 2;
  const int tr_q = lane & 3;
  const int kt_lane = ((trG >> 1) * 8 + tr_m) * 64 + 32 * (trG & 1) + 8 * tr_q;
  // V^T reads (P V): row t32, chunk half ^ ((t32>>2)&3) for c = 0; c = 1 flips
  // bit 1 of the chunk, i.e. byte offset ^ 32
  const int vt_lane = t32 * 64 + 16 * (half ^ ((t32 >> 2) & 3));
  // identity fragments: row key (t32), slot half*8+e of chunk cb <-> key cb*16+half*8+e
  Frag<bf16> idf[2];
#pragma unroll
  for (int cb = 0; cb < 2; ++cb)
#pragma unroll
    for (int e = 0; e < 8; ++e)
      idf[cb].v[e] = (bf16)(t32 == cb * 16 + half * 8 + e ? 1.0f : 0.0f);
  const bf16* brow = ws.bias + ((int64_t)(b * H + h) * Np + q0 + t32) * Np + half * 8;
  Frag<bf16> bfr[2];  // bias fragments of the next S tile to issue
  auto load_bias = [&](int t) {
    bfr[0].load(brow + t * 32);
    bfr[1].load(brow + t * 32 + 16);
  };
  // S^T - m of 32-key tile t: the accumulation starts from negm = -m_use in
  // every register, then adds I.Bias^T and K Q^T.
  f32x16 negm = zero16();
  auto s_tile = [&](int t) {
    f32x16 s = __builtin_amdgcn_mfma_f32_32x32x16_bf16(idf[0].v, bfr[0].v, negm, 0, 0, 0);
    mma(s, idf[1], bfr[1]);
    // sub-block t&1 of this head's K^T; row d = m*16 + (trG>>1)*8 + hh*4 +
    // tr_m, keys 16*(trG&1) + 4*tr_q: one base plus constant offsets
    const char* kt_base = ring[(t >> 1) % NS] + h * HEAD_BYTES + (t & 1) * 2048 + kt_lane;
#pragma unroll
    for (int m = 0; m < 2; ++m) {
      s16x4 part[2];
#pragma unroll
      for (int hh = 0; hh < 2; ++hh) part[hh] = lds_read_tr16(kt_base + (m * 16 + hh * 4) * 64);
      typedef short s16x8 __attribute__((ext_vector_type(8)));
      const s16x8 v8 = {part[0][0], part[0][1], part[0][2], part[0][3],
                        part[1][0], part[1][1], part[1][2], part[1][3]};
      Frag<bf16> kf;
      kf.v = __builtin_bit_cast(bf16x8, v8);
      mma(s, kf, qf[m]);
    }
    return s;
  };

  const int nkb = (N + KB - 1) / KB;
  const int ntiles = 2 * nkb;
  static_assert(NW * 2048 <= STAGE_BYTES && NS >= 2, "q / gate tiles fit in one ring stage");
  issue_stage(0, 0);
  issue_cq(q_src, 1);
  load_bias(0);
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  typedef short s16x8 __attribute__((ext_vector_type(8)));
#pragma unroll
  for (int m = 0; m < 2; ++m) {
    const s16x4 lo = read_cq4(1, m * 16 + half * 8), hi = read_cq4(1, m * 16 + half * 8 + 4);
    const s16x8 v8 = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
    qf[m].v = __builtin_bit_cast(bf16x8, v8);
  }
  barrier_only();  // every wave has read its q tile: stage 1 is free
  // stage 1, or (a single key block) the gate tile, into the free stage
  if (nkb > 1) issue_stage(1, KB);
  else issue_cq(g_src, 1);

  typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
  const bf16x2_t ones2 = {(bf16)1.0f, (bf16)1.0f};
  f32x16 o = zero16();
  float m_ref = -INFINITY, l_run = 0.f;
  float m_use = 0.f;  // the reference subtracted from the scores: m_ref, or 0 while m_ref = -inf
  // The part of m_use subtracted inside S (negm = -m_in): m_use while
  // |m_use| < kFar, else 0.  A reference set by masked keys only (about
  // -inf log2 e) folded into the fp32 accumulation would round the logits of
  // the valid keys that follow to multiples of its ulp; such a lane
  // subtracts it on the VALU instead (a rare path: a row whose running
  // maximum so far comes from masked keys).
  constexpr float kFar = 4096.f;
  float m_in = 0.f;
  for (int t = 0; t < ntiles; ++t) {
    const bool opens = t > 0 && (t & 1) == 0;  // tile t opens key block t/2
    if (opens) {
      __builtin_amdgcn_s_waitcnt(0);      // stage t/2 and the bias of tile t landed
      __syncthreads();                    // ... for every wave; block t/2-2 fully consumed
    }
    f32x16 sc = s_tile(t);
    if (t + 1 < ntiles) load_bias(t + 1);
    // The next block's copy goes out after the bias of tile t+1: loads
    // complete in issue order, so waiting for that bias does not wait for it.
    if (opens && (t >> 1) + 1 < nkb) issue_stage(((t >> 1) + 1) % NS, ((t >> 1) + 1) * KB);
    // the last block opens: the gate tile goes into the stage it leaves free
    if (opens && (t >> 1) + 1 == nkb) issue_cq(g_src, nkb % NS);
    const int cur = (t >> 1) % NS;
    // padding keys of tile t take no weight, masked keys their mask bias
    // (none at all in a clean row: no LDS read).  For a row whose keys are
    // all masked the scores follow the reference's fp32 arithmetic: with
    // inf = 1e9 they round to one value, and the row attends uniformly.
    const unsigned kx = row_clean ? 0u : (kpad[t] | kmask[t]);
    if (kx != 0u) {
      const unsigned kp = kpad[t] >> (4 * half), km = kmask[t] >> (4 * half);
      const unsigned kf = kfrac[t];
#pragma unroll
      for (int g = 0; g < 4; ++g)
#pragma unroll
        for (int rr = 0; rr < 4; ++rr) {
          float add = ((km >> (8 * g + rr)) & 1u) ? madd0 : 0.f;
          if (kf != 0u && ((kf >> (8 * g + 4 * half + rr)) & 1u))
            add = (inf * (mrow[(int64_t)(32 * t + 8 * g + 4 * half + rr) * mks] - 1.f)) * kLog2e;
          sc[4 * g + rr] = ((kp >> (8 * g + rr)) & 1u) ? -INFINITY : sc[4 * g + rr] + add;
        }
    }
    // sc holds s - m_in; the reference max m_ref moves only when a score
    // exceeds it by more than kRescale
    float mt = fmaxf(fmaxf(sc[0], sc[1]), sc[2]);
#pragma unroll
    for (int e = 3; e < 15; e += 2) mt = fmaxf(fmaxf(mt, sc[e]), sc[e + 1]);
    mt = fmaxf(mt, sc[15]);
    mt = lane_pair_max(mt) + m_in;        // the tile max of s
    if (__ballot(mt > m_ref + kRescale) != 0ull) {
      const float m_new = fmaxf(m_ref, mt);
      const float alpha = (m_new == -INFINITY) ? 1.f : __builtin_amdgcn_exp2f(m_ref - m_new);
      l_run *= alpha;
#pragma unroll
      for (int e = 0; e < 16; ++e) o[e] *= alpha;
      m_ref = m_new;
      m_use = (m_ref == -INFINITY) ? 0.f : m_ref;
      const float m_in_new = fabsf(m_use) < kFar ? m_use : 0.f;
      const float shift = m_in - m_use;
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        sc[e] += shift;
        negm[e] = -m_in_new;
      }
      m_in = m_in_new;
    } else if (__ballot(m_in != m_use) != 0ull) {
      // a lane whose reference stays beyond kFar: its scores are raw
#pragma unroll
      for (int e = 0; e < 16; ++e) sc[e] += m_in - m_use;
    }
    // sub-block t&1 of this head's V^T, row t32
    const char* vt_base = ring[cur] + (H + h) * HEAD_BYTES + (t & 1) * 2048;
#pragma unroll
    for (int c = 0; c < 2; ++c) {
      Frag<bf16> pf, vf;
#pragma unroll
      for (int e = 0; e < 8; ++e) pf.v[e] = (bf16)__builtin_amdgcn_exp2f(sc[8 * c + e]);
      // row sum over the bf16 probabilities that enter P V
#pragma unroll
      for (int e = 0; e < 8; e += 2) {
        const bf16x2_t pp = {pf.v[e], pf.v[e + 1]};
        l_run = __builtin_amdgcn_fdot2_f32_bf16(pp, ones2, l_run, false);
      }
      // keys 16c + 8*half .. +8 of the sub-block: chunk (2c + half) ^ ((t32>>2)&3)
      vf.load(reinterpret_cast<const bf16*>(vt_base + (c ? (vt_lane ^ 32) : vt_lane)));
      mma(o, vf, pf);
    }
  }
  const float inv = 1.0f / lane_pair_sum(l_run);
  // Epilogue.  Every global load it needs (the W_o fragments and the
  // residual rows of this wave's output tile, the gate) is issued here,
  // before the first store: vmcnt counts stores too, so a load issued after
  // a store is only waited for together with that store.
  constexpr int NT = CIN / 32;
  static_assert(QT * NT == H * QT, "one output tile per wave");
  const int oq = wave / NT, nt = wave % NT;
  Frag<bf16> wof[CH / 16];
  if constexpr (!WO_LDS) {
#pragma unroll
    for (int ks = 0; ks < CH / 16; ++ks) load_wfrag<bf16>(wof[ks], w.w_o, nt, ks, CH / 16);
  }
  const int q_out = qb * QB + oq * 32 + t32;
  const bool q_ok = q_out < N;
  const int64_t pair_out =
      ((int64_t)b * N + (starting ? r : (q_ok ? q_out : 0))) * N + (starting ? (q_ok ? q_out : 0) : r);
  f32x4 bo[4];
#pragma unroll
  for (int g = 0; g < 4; ++g) bo[g] = *reinterpret_cast<const f32x4*>(w.b_o + nt * 32 + 8 * g + 4 * half);
  bf16x4 xres[4];
  if (residual) {
#pragma unroll
    for (int g = 0; g < 4; ++g)
      xres[g] = *reinterpret_cast<const bf16x4*>(x + pair_out * CIN + nt * 32 + 8 * g + 4 * half);
  }
  // this lane's gate values (channel-major, like q)
  bf16x4 gpre[4];
  __builtin_amdgcn_s_waitcnt(0);  // this wave's gate tile has landed (wave-local region)
#pragma unroll
  for (int g = 0; g < 4; ++g) gpre[g] = __builtin_bit_cast(bf16x4, read_cq4(nkb % NS, 8 * g + 4 * half));

  // o * gate for all heads, staged as [query][CH] over the ring
  __syncthreads();
  bf16* os = reinterpret_cast<bf16*>(&ring[0][0]);
#pragma unroll
  for (int g = 0; g < 4; ++g) {
    const int d0 = 8 * g + 4 * half;
    const bf16x4 gv = gpre[g];
    store4(os + (qt * 32 + t32) * OP + h * HD + d0, o[4 * g] * inv * (float)gv[0],
           o[4 * g + 1] * inv * (float)gv[1], o[4 * g + 2] * inv * (float)gv[2],
           o[4 * g + 3] * inv * (float)gv[3]);
  }
  __syncthreads();
  // output projection: wave -> (query tile oq, output tile nt)
  {
    Frag<bf16> of[CH / 16];
#pragma unroll
    for (int ks = 0; ks < CH / 16; ++ks) of[ks].load(os + (oq * 32 + t32) * OP + half * (CH / 2) + ks * 8);
    f32x16 acc = zero16();
#pragma unroll
    for (int ks = 0; ks < CH / 16; ++ks) {
      if constexpr (WO_LDS) load_wfrag_lds(wof[ks], wo_l, nt, ks, CH / 16);
      mma(acc, wof[ks], of[ks]);
    }
    if (q_ok) {
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int c0 = nt * 32 + 8 * g + 4 * half;
        float v[4];
#pragma unroll
        for (int rr = 0; rr < 4; ++rr) {
          v[rr] = acc[4 * g + rr] + bo[g][rr];
          if (residual) v[rr] += (float)xres[g][rr];
        }
        store4(out + pair_out * CIN + c0, v[0], v[1], v[2], v[3]);
      }
    }
  }
}

// ---------------------------------------------------------------------------
// 3d. bf16 flash kernel, one block per (row, head), for Np <= NPM (1024).
//   * K^T and V^T of the row and head (2 x 32 x Np bf16, 64 KiB at Np = 512)
//     are copied into LDS once, with direct global->LDS loads, and stay there
//     for the whole block: after one barrier the key loop runs without any.
//     Layout: [kind][key tile t][32 d rows][64 bytes]; K^T rows unswizzled,
//     V^T chunk p of row d at physical chunk p ^ ((d>>2)&3) (the read
//     patterns of the module kernel above).
//   * NW waves (8, or 16 at Np = 1024); wave w attends query tiles w,
//     w+NW, ... in turn.  Each
//     query tile: q copied into the wave's 2 KiB LDS region and read back
//     transposed, the gate tile copied into the same region behind it, then
//     the key loop (bf16 bias tiles prefetched two tiles ahead and widened
//     into the S^T accumulator, the next tile's K fragments read a tile
//     ahead), then o / l * gate stored into og in the
//     output projection's fragment order (og_frag_off).  The next tile's q
//     copy is issued before those stores.
//   * The excluded-key bits of the row are kept in one VGPR (lane t: key
//     tile t) and read with v_readlane per tile.  The prologue's bias pass
//     wrote them (one word and one flags word per key tile): the block loads
//     64 contiguous bytes instead of the row's mask values, which for the
//     ending node are a column of the mask, one cache line per key, read by
//     every wave of every head's block.
//   * Blocks run head-major, so the blocks of one XCD read one or two heads'
//     triangle bias.  That bias (1 MiB per head at Np = 512) is re-read by
//     every row's block, while K^T, V^T, q and the gate are read once: their
//     copies carry the non-temporal hint so they do not evict the bias from
//     L2 (150 -> 141 us standalone at N = 512; with every bias load hitting a
//     64 KiB window the kernel takes 133 us).
// The output projection (W_o, b_o, residual) runs in triattn_out_kernel.
// ---------------------------------------------------------------------------
// NW waves per block: 8 at Np <= 512 (two blocks per CU), 16 at Np = 1024,
// where K^T and V^T take 128 KiB of LDS and one block fills the CU (16 x 2 KiB
// of staging beside them: 160 KiB), so the CU still holds 16 waves.
template <int NPM, int NW>
__global__ __launch_bounds__(64 * NW) __attribute__((amdgpu_waves_per_eu(4))) void triattn_flash_rh_kernel(
    const float* __restrict__ mask, AttnWs<bf16> ws, int N, int Np, int starting, int r0, int nrows,
    float inf) {
  constexpr int H = 4, CH = H * HD;
  static_assert(2 * NPM / 32 * 2048 + NW * 2048 <= 160 * 1024, "K^T, V^T and staging in one CU's LDS");
  constexpr int NTM = NPM / 32;       // key tiles at most
  constexpr float kRescale = 8.0f;    // lazy-rescale threshold (log2 units)
  static_assert(NTM <= 64, "excluded-key bits: one word per lane");
  __shared__ __attribute__((aligned(1024))) char kv[2 * NTM * 2048];
  __shared__ __attribute__((aligned(1024))) char stg[NW][2048];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int half = lane >> 5;
  const int t32 = lane & 31;
  const int nt = Np / 32;             // key tiles (even: Np is a multiple of 128)
  const int nq = (N + 31) / 32;       // query tiles holding real queries
  const int64_t per_h = (int64_t)gridDim.x / H;
  const int64_t lin = xcd_remap(blockIdx.x, gridDim.x);
  const int h = (int)(lin / per_h);
  const int64_t rem = lin - h * per_h;
  const int b = (int)(rem / nrows);
  const int r = r0 + (int)(rem - (int64_t)b * nrows);
  const int64_t rowbase = ws.row(b, r);

  // K^T / V^T of (row, head): 4 * nt copies of 1 KiB (kind, tile, row half)
  {
    const bf16* kbase = ws.k + (rowbase * H + h) * (int64_t)HD * Np;
    const bf16* vbase = ws.vt + (rowbase * H + h) * (int64_t)HD * Np;
    // tiled layout: key tile t is [32 d][32 keys], 2 KiB contiguous
    const uint32_t ln = (uint32_t)lane;
    const uint32_t rowoff = (ln >> 2) * 64;
    const uint32_t voff_k = rowoff + (ln & 3) * 16;
    const uint32_t voff_v = rowoff + (((ln & 3) ^ ((ln >> 4) & 3)) * 16);
    const uint32_t kv_lds = lds_addr(kv);
    for (int c = wave; c < 4 * nt; c += NW) {
      const int kind = c >= 2 * nt;
      const int cr = c - kind * 2 * nt;
      const int t = cr >> 1, rh = cr & 1;
      const bf16* src = (kind ? vbase : kbase) + t * 1024 + rh * 512;
      g2lds16_sv_nt(src, kind ? voff_v : voff_k, kv_lds + ((kind * NTM + t) * 2 + rh) * 1024);
    }
  }

  // Masked keys of this row (mask != 1), one bit per key (bit j of lane t's
  // word is key 32t + j), from the row's mask words (written with the bias).
  // They take the reference's additive bias inf * (mask - 1), here in log2
  // units; padding keys (k >= N, the tail of the last tiles) take no weight.
  // row_frac: some mask value is neither 0 nor 1, whose bias is then
  // computed from the value (mrow).  A row where every key carries a mask
  // bias goes straight to the exact pass, where the reference's fp32
  // arithmetic is followed (with inf = 1e9 every score of such a row rounds
  // to the same value: uniform attention).  Wave-uniform: every wave reads
  // the same row.
  const float* mrow = mask ? mask + (int64_t)b * N * N + (starting ? (int64_t)r * N : r) : nullptr;
  const int64_t mks = starting ? 1 : N;
  const int64_t mwi = ((int64_t)b * Np + r) * (Np / 32) + lane;
  const uint32_t kmv = lane < nt ? ws.mbits[mwi] : 0u;
  const int mfl = lane < nt ? ws.mflags[mwi] : 0;
  const bool row_valid = __ballot((mfl & 1) != 0) != 0ull;
  const bool row_frac = __ballot((mfl & 2) != 0) != 0ull;
  const float madd0 = -inf * kLog2e;  // the bias of a key with mask == 0

  const uint32_t stg_lds = lds_addr(stg[wave]);
  char* const sw = stg[wave];
  // q or gate tile [32 channels][32 queries] (2 KiB contiguous in the tiled
  // layout) -> the wave's region, 64-byte rows; copy j moves channels
  // 16j .. 16j+15, lane l takes channel 16j + l/4, queries 8*(l%4) .. +7
  auto issue_cq = [&](const bf16* src) {
    const uint32_t ln = (uint32_t)(lane + opaque_zero());
    const uint32_t voff = ln * 16;
#pragma unroll
    for (int j = 0; j < 2; ++j) g2lds16_sv_nt(src + j * 512, voff, stg_lds + j * 1024);
  };
  // channels c0 .. c0+3 of this lane's query t32 (transposing read); ln is
  // the lane id through opaque_zero, so that these per-lane addresses are
  // recomputed where they are used instead of held across the key loop
  auto read_cq4 = [&](int ln, int c0) {
    const int i = ln & 15;
    return lds_read_tr16(sw + (c0 + (i >> 2)) * 64 + (16 * ((ln >> 4) & 1) + 4 * (i & 3)) * 2);
  };
  const bf16* q_row = ws.q + ((rowbase * H + h) * HD) * (int64_t)Np;
  const bf16* g_row = ws.gate + (rowbase * CH + h * HD) * (int64_t)Np;
  const bf16* b_head = ws.biasfr + (int64_t)(b * H + h) * Np * Np;  // wave-uniform

  // K fragments (transposing reads of K^T) and V^T fragments: per-lane offsets
  const int trG = lane >> 4;
  const int kt_lane = ((trG >> 1) * 8 + ((lane & 15) >> 2)) * 64 + 32 * (trG & 1) + 8 * (lane & 3);
  const int vt_lane = t32 * 64 + 16 * (half ^ ((t32 >> 2) & 3));

  typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
  typedef short s16x8 __attribute__((ext_vector_type(8)));
  const bf16x2_t ones2 = {(bf16)1.0f, (bf16)1.0f};
  // Bias tile t of query tile q0 (bf16) in the S^T accumulator layout:
  // register 4g + rr <-> key 32t + 8g + 4*half + rr, stored in that order
  // (bias_frag_off): 2 loads of 1 KiB contiguous per wave (a wave-uniform
  // base plus a 32-bit per-lane byte offset, the saddr form), widened to
  // fp32 where the tile's S accumulation starts.
  const uint32_t b_lane = (uint32_t)lane * 16;
  auto load_bias = [&](uint4* dst, int q0, int t) {
    const uint32_t off = b_lane + (uint32_t)(((q0 >> 5) * nt + t) * 2048);
#pragma unroll
    for (int sl = 0; sl < 2; ++sl)
      dst[sl] = *reinterpret_cast<const uint4*>(reinterpret_cast<const char*>(b_head) + off + 1024 * sl);
  };
  auto widen_bias = [](f32x16& dst, const uint4* p) {
#pragma unroll
    for (int sl = 0; sl < 2; ++sl) {
      const uint32_t d[4] = {p[sl].x, p[sl].y, p[sl].z, p[sl].w};
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        dst[8 * sl + 2 * k] = __uint_as_float(d[k] << 16);
        dst[8 * sl + 2 * k + 1] = __uint_as_float(d[k] & 0xffff0000u);
      }
    }
  };
  // K fragments of key tile t (transposing reads of K^T)
  auto k_read = [&](int t, Frag<bf16>* kf) {
    const char* kt_base = kv + t * 2048 + kt_lane;
#pragma unroll
    for (int m = 0; m < 2; ++m) {
      const s16x4 p0 = lds_read_tr16(kt_base + (m * 16) * 64);
      const s16x4 p1 = lds_read_tr16(kt_base + (m * 16 + 4) * 64);
      const s16x8 v8 = {p0[0], p0[1], p0[2], p0[3], p1[0], p1[1], p1[2], p1[3]};
      kf[m].v = __builtin_bit_cast(bf16x8, v8);
    }
  };
  // s += K Q^T for key tile t (s holds the bias tile: S^T in log2 units)
  auto s_mma = [&](f32x16& s, const Frag<bf16>* kf, const Frag<bf16>* qf) {
#pragma unroll
    for (int m = 0; m < 2; ++m) mma(s, kf[m], qf[m]);
  };
  auto s_tile = [&](int t, f32x16& s, const Frag<bf16>* qf) {
    Frag<bf16> kf[2];
    k_read(t, kf);
    s_mma(s, kf, qf);
  };
  // padding keys of tile t take no weight, masked keys their mask bias;
  // FRAC: mask values other than 0 are read back for their bias (only the
  // exact pass runs rows with such values)
  auto mask_tile = [&](int t, f32x16& sc, auto frac_tag) {
    constexpr bool FRAC = decltype(frac_tag)::value;
    const unsigned km_t = __builtin_amdgcn_readlane(kmv, t);
    const int nin = N - 32 * t;  // keys of tile t below N
    if (km_t != 0u || nin < 32) {
      // this lane's keys j = 8g + 4*half + rr: bits 8g + rr after the shift
      const int sh = 4 * (lane >> 5);
      const unsigned km = km_t >> sh;
#pragma unroll
      for (int g = 0; g < 4; ++g)
#pragma unroll
        for (int rr = 0; rr < 4; ++rr) {
          const bool mk = __builtin_amdgcn_ubfe(km, 8 * g + rr, 1);
          float add = mk ? madd0 : 0.f;
          if constexpr (FRAC) {
            if (row_frac && mk) add = (inf * (mrow[(int64_t)(32 * t + 8 * g + sh + rr) * mks] - 1.f)) * kLog2e;
          }
          sc[4 * g + rr] = 8 * g + sh + rr >= nin ? -INFINITY : sc[4 * g + rr] + add;
        }
    }
  };
  const std::false_type kBinary;
  const std::true_type kFrac;
  // the max-free pass runs when some key has no mask bias and every bias is
  // inf * (0 - 1)
  const bool fast_ok = row_valid && !row_frac;
  // P = 2^sc (bf16), l += row sums of P, O^T += V^T P^T
  auto pv_tile = [&](int t, const f32x16& sc, f32x16& o, float& l_run) {
    const char* vt_base = kv + (NTM + t) * 2048;
#pragma unroll
    for (int c = 0; c < 2; ++c) {
      Frag<bf16> pf, vf;
#pragma unroll
      for (int e = 0; e < 8; ++e) pf.v[e] = (bf16)__builtin_amdgcn_exp2f(sc[8 * c + e]);
#pragma unroll
      for (int e = 0; e < 8; e += 2) {
        const bf16x2_t pp = {pf.v[e], pf.v[e + 1]};
        l_run = __builtin_amdgcn_fdot2_f32_bf16(pp, ones2, l_run, false);
      }
      vf.load(reinterpret_cast<const bf16*>(vt_base + (c ? (vt_lane ^ 32) : vt_lane)));
      mma(o, vf, pf);
    }
  };

  // Bias of the next KB S tiles, prefetched KB - 1 tiles ahead (bf16, 8
  // registers a tile; four tiles ahead measured slower); S^T accumulates on
  // the widened bias.  Each tile's loads go out unconditionally (the
  // last KB of a query tile fetch the first KB of the wave's next query
  // tile, or again the current one at the end), so the compiler's waits
  // count them exactly.
  constexpr int KB = 2;
  // Epilogue of query tile q0: o / l * gate, stored into og in the output
  // projection's B-fragment order (og_frag_off): this head's 32 channels are
  // 4 chunks of 8; the two half-waves trade quads (v_permlane32_swap) so that
  // the lower one writes chunks 0-1 and the upper one chunks 2-3, each store
  // 32 lanes x 16 bytes contiguous.  next_q: the q tile to copy into the
  // wave's region before the stores (null: none).
  const int64_t og_tiles = rowbase * (int64_t)nt;  // og tile index of (row, query tile 0)
  auto finish = [&](int q0, const f32x16& o, float l_tot, const bf16* next_q) {
    const float inv = 1.0f / l_tot;
    const int lne = lane + opaque_zero();
    const int ehalf = lne >> 5;
    // The gate tile has landed (wave-local region): it was copied before
    // every bias load of this query tile, and at most the last KB tiles'
    // bias loads (the next query tile's first) may still be outstanding;
    // the exact pass waits for each of its own loads.
    __builtin_amdgcn_s_waitcnt(vmcnt_imm<2 * KB>());
    bf16x4 gv[4];
#pragma unroll
    for (int g = 0; g < 4; ++g) gv[g] = __builtin_bit_cast(bf16x4, read_cq4(lne, 8 * g + 4 * ehalf));
    // quad g of this lane: channels 8g + 4*half .. +3 of query t32
    uint32_t px[4], py[4];
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      px[g] = pack_bf16x2(o[4 * g] * inv * (float)gv[g][0], o[4 * g + 1] * inv * (float)gv[g][1]);
      py[g] = pack_bf16x2(o[4 * g + 2] * inv * (float)gv[g][2], o[4 * g + 3] * inv * (float)gv[g][3]);
    }
    // lower half receives the upper's quads of chunks 0, 1; the upper half
    // the lower's quads of chunks 2, 3
    const auto s0x = __builtin_amdgcn_permlane32_swap(px[0], px[2], false, false);
    const auto s0y = __builtin_amdgcn_permlane32_swap(py[0], py[2], false, false);
    const auto s1x = __builtin_amdgcn_permlane32_swap(px[1], px[3], false, false);
    const auto s1y = __builtin_amdgcn_permlane32_swap(py[1], py[3], false, false);
    const bool up = ehalf != 0;
    const uint4 cA = up ? make_uint4(s0x[0], s0y[0], px[2], py[2]) : make_uint4(px[0], py[0], s0x[1], s0y[1]);
    const uint4 cB = up ? make_uint4(s1x[0], s1y[0], px[3], py[3]) : make_uint4(px[1], py[1], s1x[1], s1y[1]);
    __builtin_amdgcn_s_waitcnt(0xC07F);  // gate read: the region is free for the next q copy
    if (next_q) issue_cq(next_q);
    const int ks = (h & 1) * 4 + (up ? 2 : 0);  // chunk of cA; cB is ks + 1
    const uint32_t o_off = (uint32_t)og_frag_off(og_tiles + (q0 >> 5), ks, (h >> 1) * 32 + (lne & 31)) * 2;
    *reinterpret_cast<uint4*>(reinterpret_cast<char*>(ws.og) + o_off) = cA;
    *reinterpret_cast<uint4*>(reinterpret_cast<char*>(ws.og) + o_off + 1024) = cB;
  };

  uint4 bq[KB][2];
  // K fragments of the fast pass's next tile, read one tile ahead (the last
  // tile of a query tile reads tile 0 for the next query tile)
  Frag<bf16> kn[2];
  int qt = wave;
  if (qt < nq) {
    issue_cq(q_row + qt * 1024);
    if (fast_ok) {
#pragma unroll
      for (int u = 0; u < KB; ++u) load_bias(bq[u], qt * 32, u);
    }
  }
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();  // K^T / V^T resident for every wave
  k_read(0, kn);
  for (; qt < nq; qt += NW) {
    const int q0 = qt * 32;
    const int q0n = (qt + NW < nq ? qt + NW : qt) * 32;  // the query tile to prefetch for
    // this tile's q copy landed: behind it are, after the first tile, the
    // previous tile's og stores (2)
    if (qt != wave) __builtin_amdgcn_s_waitcnt(vmcnt_imm<2>());
    Frag<bf16> qf[2];
    const int lnq = lane + opaque_zero();
#pragma unroll
    for (int m = 0; m < 2; ++m) {
      const s16x4 lo = read_cq4(lnq, m * 16 + half * 8), hi = read_cq4(lnq, m * 16 + half * 8 + 4);
      const s16x8 v8 = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
      qf[m].v = __builtin_bit_cast(bf16x8, v8);
    }
    __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): q read back, the region is free
    issue_cq(g_row + qt * 1024);                // the gate tile lands behind the key loop

    // Fast pass: P = 2^s with no running maximum.  Exact (softmax is shift
    // invariant, and fp32 / bf16 keep relative precision) while every 2^s
    // stays in range; checked at the end through l, else the exact pass runs.
    f32x16 o = zero16();
    float l_run = 0.f;
    for (int t = 0; fast_ok && t < nt; t += KB) {
#pragma unroll
      for (int u = 0; u < KB; ++u) {
        f32x16 sc;
        widen_bias(sc, bq[u]);
        s_mma(sc, kn, qf);
        k_read(t + u + 1 < nt ? t + u + 1 : 0, kn);
        mask_tile(t + u, sc, kBinary);
        pv_tile(t + u, sc, o, l_run);
        const bool wrap = t + u + KB >= nt;
        load_bias(bq[u], wrap ? q0n : q0, wrap ? t + u + KB - nt : t + u + KB);
        // one sub-tile at a time: interleaving them would need several S
        // tiles and their fragments live at once
        __builtin_amdgcn_sched_barrier(0);
      }
    }
    float l_tot = lane_pair_sum(l_run);
    // In range: the largest term 2^max(s) is within [2^-69, 2^64], so no P
    // overflows and no term that underflows matters.  Tested on the bits:
    // positive floats order as unsigned integers, and a NaN, a zero, a
    // negative value or infinity all fall outside.
    if (!fast_ok || __ballot(!l_in_range(l_tot)) != 0ull) {
      // Exact pass: online softmax with a running maximum, lazily moved (only
      // when a tile exceeds it by more than kRescale), bias loaded per tile.
      o = zero16();
      l_run = 0.f;
      float m_ref = -INFINITY, m_use = 0.f;
      for (int t = 0; t < nt; ++t) {
        f32x16 sc;
        {
          uint4 bp[2];
          load_bias(bp, q0, t);
          widen_bias(sc, bp);
        }
        s_tile(t, sc, qf);
        mask_tile(t, sc, kFrac);
        // the tile max of the raw scores; the reference is subtracted
        // afterwards.  (Subtracted first, a reference set by a tile of
        // masked keys only, about -inf log2 e, would round the logits of the
        // valid keys that follow to multiples of its fp32 ulp.)
        float mt = fmaxf(fmaxf(sc[0], sc[1]), sc[2]);
#pragma unroll
        for (int e = 3; e < 15; e += 2) mt = fmaxf(fmaxf(mt, sc[e]), sc[e + 1]);
        mt = lane_pair_max(fmaxf(mt, sc[15]));
        if (__ballot(mt > m_ref + kRescale) != 0ull) {
          const float m_new = fmaxf(m_ref, mt);
          const float alpha = (m_new == -INFINITY) ? 1.f : __builtin_amdgcn_exp2f(m_ref - m_new);
          l_run *= alpha;
#pragma unroll
          for (int e = 0; e < 16; ++e) o[e] *= alpha;
          m_ref = m_new;
          m_use = (m_ref == -INFINITY) ? 0.f : m_ref;
        }
#pragma unroll
        for (int e = 0; e < 16; ++e) sc[e] -= m_use;
        pv_tile(t, sc, o, l_run);
      }
      l_tot = lane_pair_sum(l_run);
    }
    finish(q0, o, l_tot, qt + NW < nq ? q_row + (qt + NW) * 1024 : nullptr);
  }
}

// ---------------------------------------------------------------------------
// 3e. Output projection of the (row, head) flash path:
//     out[pair] = og[row][q] . W_o^T + b_o (+ x[pair]) at the source pair of
//     (row, q).  Persistent blocks of 8 waves (two per CU), W_o (packed, 32
//     KiB) and b_o in LDS; one tile = 32 consecutive queries of one row.
//   * og arrives in fragment order (og_frag_off): 8 loads of 1 KiB
//     contiguous, issued with the residual rows at the start of the tile
//     (four waves per SIMD hide their latency).
//   * The result is transposed through the wave's 4 KiB LDS region in two
//     halves of 64 channels (bf16 update, rows of 128 bytes, chunk c of row q
//     at physical chunk c ^ (q & 7)), then every lane adds 8 residual
//     channels and stores 16 bytes: 8 lanes write one 128-byte line, for the
//     starting node's consecutive pairs and the ending node's strided ones.
//     The update is rounded to bf16 before the residual add, as the module's
//     bf16 output is before the caller's residual add.
// ---------------------------------------------------------------------------
template <int CIN>
__global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(4))) void triattn_out_kernel(const bf16* __restrict__ x, bf16* __restrict__ out,
                                                          TriAttnPacked<bf16> w, AttnWs<bf16> ws, int N,
                                                          int Np, int starting, int residual, int r0,
                                                          int nrows, int64_t ntiles) {
  constexpr int CH = 4 * HD;
  constexpr int KC = CH / 16;   // k chunks over c_h
  constexpr int NTO = CIN / 32; // output tiles of 32 channels
  static_assert(CIN == 128 && NTO == 4, "two halves of 64 output channels");
  __shared__ __attribute__((aligned(1024))) bf16 wl[NTO * KC * 512];
  __shared__ __attribute__((aligned(16))) float bl[CIN];
  __shared__ __attribute__((aligned(1024))) char stg[8][4096];
  copy_to_lds_async(wl, w.w_o, (int)sizeof(wl));
  for (int t = threadIdx.x; t < CIN; t += blockDim.x) bl[t] = w.b_o[t];
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  const int lane = threadIdx.x & 63;
  const int wave = wave_id();
  const int half = lane >> 5;
  const int t32 = lane & 31;
  char* const sw = stg[wave];
  const int qtiles = (N + 31) / 32;
  const int ntq = Np / 32;  // og tiles per workspace row
  const int64_t stride = (int64_t)gridDim.x * 8;
  auto og_tile = [&](int64_t tile) {
    const int qtl = (int)(tile % qtiles);
    const int64_t br = tile / qtiles;
    const int b = (int)(br / nrows);
    const int r = r0 + (int)(br - (int64_t)b * nrows);
    return ws.row(b, r) * ntq + qtl;
  };
  auto load_og = [&](Frag<bf16>* of, int64_t tile) {
    const bf16* src = ws.og + og_frag_off(og_tile(tile), 0, lane);
#pragma unroll
    for (int ks = 0; ks < KC; ++ks) of[ks].load(src + ks * 512);
  };
  for (int64_t tile = (int64_t)blockIdx.x * 8 + wave; tile < ntiles; tile += stride) {
    const int qtl = (int)(tile % qtiles);
    const int64_t br = tile / qtiles;
    const int b = (int)(br / nrows);
    const int r = r0 + (int)(br - (int64_t)b * nrows);
    // row-pass lanes: query qq = 8i + lane/8 of the tile, 16-byte chunk lane%8
    // of a 64-channel half
    const int rq = lane >> 3, rc = lane & 7;
    const auto ors = buf_rsrc(out + (int64_t)b * N * N * CIN, (uint32_t)((int64_t)N * N * CIN * 2));
    auto pair_of = [&](int q) {  // source pair of (row r, query q), q < N
      return starting ? ((int64_t)r * N + q) : ((int64_t)q * N + r);
    };
    // residual rows of this tile (queries >= N read pair 0 and are not stored)
    uint4 xr[2][4];
    if (residual) {
#pragma unroll
      for (int hp = 0; hp < 2; ++hp)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int q = qtl * 32 + 8 * i + rq;
          const int64_t pr = q < N ? pair_of(q) : 0;
          xr[hp][i] = *reinterpret_cast<const uint4*>(x + ((int64_t)b * N * N + pr) * CIN + hp * 64 + rc * 8);
        }
    }
    Frag<bf16> cur[KC];
    load_og(cur, tile);
    const bf16* wlt = wl + opaque_zero();  // keep the W_o reads in the loop
#pragma unroll
    for (int hp = 0; hp < 2; ++hp) {
#pragma unroll
      for (int n2 = 0; n2 < 2; ++n2) {
        const int nt = 2 * hp + n2;
        Frag<bf16> f;
        load_wfrag_lds(f, wlt, nt, 0, KC);
        f32x16 acc = mma0(f, cur[0]);  // rows = outputs, columns = queries
#pragma unroll
        for (int ks = 1; ks < KC; ++ks) {
          load_wfrag_lds(f, wlt, nt, ks, KC);
          mma(acc, f, cur[ks]);
        }
        // outputs 32 n2 + 8g + 4*half .. +3 of the half, query t32
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const int c = 32 * n2 + 8 * g + 4 * half;  // channel within the half
          const f32x4 b4 = *reinterpret_cast<const f32x4*>(bl + hp * 64 + c);
          store4(reinterpret_cast<bf16*>(sw + t32 * 128 + (((c >> 3) ^ (t32 & 7)) << 4) + (c & 7) * 2),
                 acc[4 * g] + b4[0], acc[4 * g + 1] + b4[1], acc[4 * g + 2] + b4[2],
                 acc[4 * g + 3] + b4[3]);
        }
      }
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int qq = 8 * i + rq;
        uint4 v = *reinterpret_cast<const uint4*>(sw + qq * 128 + ((rc ^ (qq & 7)) << 4));
        if (residual) {
          const bf16x8 a = __builtin_bit_cast(bf16x8, v), xv = __builtin_bit_cast(bf16x8, xr[hp][i]);
          float s[8];
#pragma unroll
          for (int e = 0; e < 8; ++e) s[e] = (float)a[e] + (float)xv[e];
          v = make_uint4(pack_bf16x2(s[0], s[1]), pack_bf16x2(s[2], s[3]), pack_bf16x2(s[4], s[5]),
                         pack_bf16x2(s[6], s[7]));
        }
        const int q = qtl * 32 + qq;
        buf_store16(ors, q < N ? (uint32_t)((pair_of(q) * CIN + hp * 64 + rc * 8) * 2) : kBufSkip, v);
      }
      __builtin_amdgcn_s_waitcnt(0xC07F);  // the region is read back before the next half
    }
  }
}

// ---------------------------------------------------------------------------
// 3b. Raw attention op: relayout of q/k/v/bias, then flash per (row, head).
// ---------------------------------------------------------------------------
// src: [B][H][N][N][D]; element (b, h, a1, a2, d).  Destination row/position:
// starting (r, j) = (a1, a2); ending (r, j) = (a2, a1).
template <typename T>
__global__ void relayout_qkv_kernel(const T* __restrict__ src, T* __restrict__ dst, int B, int H,
                                    int N, int Np, int starting, int transpose_v, float scale) {
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t total = (int64_t)B * H * N * N * HD;
  if (idx >= total) return;
  const int d = (int)(idx % HD);
  int64_t t = idx / HD;
  const int a2 = (int)(t % N); t /= N;
  const int a1 = (int)(t % N); t /= N;
  const int h = (int)(t % H);
  const int b = (int)(t / H);
  const int r = starting ? a1 : a2, j = starting ? a2 : a1;
  const int64_t base = ((int64_t)b * Np + r) * H + h;
  const float v = to_f32(src[idx]) * scale;
  if (transpose_v) dst[(base * HD + d) * Np + vt_pos(j)] = cvt<T>(v);
  else dst[(base * Np + j) * HD + d] = cvt<T>(v);
}

template <typename T>
__global__ void relayout_bias_kernel(const float* __restrict__ src, T* __restrict__ dst,
                                     int B, int H, int N, int Np) {
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t total = (int64_t)B * H * N * N;
  if (idx >= total) return;
  const int k = (int)(idx % N);
  const int64_t t = idx / N;
  const int q = (int)(t % N);
  const int64_t bh = t / N;
  dst[(bh * Np + q) * Np + k] = cvt<T>(src[idx] * kLog2e);
}

template <typename T>
__global__ __launch_bounds__(64) void triattn_raw_kernel(const float* __restrict__ mask,
                                                         T* __restrict__ out, AttnWs<T> ws, int B,
                                                         int H, int N, int Np, int starting) {
  const int lane = threadIdx.x & 63;
  const int half = lane >> 5;
  const int t32 = lane & 31;
  const int qtiles = (N + 31) / 32;
  int64_t t = blockIdx.x;
  const int qt = (int)(t % qtiles); t /= qtiles;
  const int h = (int)(t % H); t /= H;
  const int r = (int)(t % N);
  const int b = (int)(t / N);
  const int q0 = qt * 32;
  const int64_t rowbase = (int64_t)b * Np + r;
  MaskView mv;
  mv.m = mask + (int64_t)b * N * N + (starting ? (int64_t)r * N : r);
  mv.row_stride = 0;
  mv.key_stride = starting ? 1 : N;
  mv.inf = 1e9f;  // the reference's default TriangleAttention(inf=1e9)
  const f32x16 o = flash_row_head<T>(ws.q + (rowbase * H + h) * Np * HD,
                                     ws.k + (rowbase * H + h) * Np * HD,
                                     ws.vt + (rowbase * H + h) * HD * (int64_t)Np,
                                     ws.bias + ((int64_t)b * H + h) * Np * Np, mv, q0, N, Np);
  const int q = q0 + t32;
  if (q >= N) return;
  const int p0 = starting ? r : q, p1 = starting ? q : r;
  T* dst = out + (((int64_t)b * N + p0) * N + p1) * (int64_t)(H * HD) + h * HD;
#pragma unroll
  for (int g = 0; g < 4; ++g) {
    const int d0 = 8 * g + 4 * half;
    store4(dst + d0, o[4 * g], o[4 * g + 1], o[4 * g + 2], o[4 * g + 3]);
  }
}

template <typename T>
static int raw_attention(const void* q, const void* k, const void* v, const float* bias,
                         const float* mask, float scale, void* out, int64_t B, int64_t H,
                         int64_t N, void* ws, int starting, hipStream_t st) {
  const int Np = (int)attn_pad(N);
  Carve cv(ws, SIZE_MAX);
  AttnWs<T> w = carve_attn_ws<T>(cv, B, Np, (int)H, 0);
  // zero the padded workspace so padded keys/queries read finite values
  int rc = launch_zero(w.q, (size_t)((char*)(w.bias + B * H * (int64_t)Np * Np) - (char*)w.q), st);
  if (rc) return rc;
  const int64_t total = B * H * N * N * HD;
  const unsigned g1 = (unsigned)((total + 255) / 256);
  relayout_qkv_kernel<T><<<g1, 256, 0, st>>>((const T*)q, w.q, (int)B, (int)H, (int)N, Np, starting, 0, scale * kLog2e);
  GTK_LAUNCH_CHECK();
  relayout_qkv_kernel<T><<<g1, 256, 0, st>>>((const T*)k, w.k, (int)B, (int)H, (int)N, Np, starting, 0, 1.f);
  GTK_LAUNCH_CHECK();
  relayout_qkv_kernel<T><<<g1, 256, 0, st>>>((const T*)v, w.vt, (int)B, (int)H, (int)N, Np, starting, 1, 1.f);
  GTK_LAUNCH_CHECK();
  const int64_t tb = B * H * N * N;
  relayout_bias_kernel<T><<<(unsigned)((tb + 255) / 256), 256, 0, st>>>(bias, w.bias, (int)B, (int)H, (int)N, Np);
  GTK_LAUNCH_CHECK();
  const int64_t blocks = B * N * H * ((N + 31) / 32);
  GTK_REQUIRE(blocks < (1ll << 31), GTK_EUNSUPPORTED, "attention grid too large");
  {
    StageTimer timer("triattn_raw", st);
    triattn_raw_kernel<T><<<(unsigned)blocks, 64, 0, st>>>(mask, (T*)out, w, (int)B, (int)H, (int)N, Np, starting);
  }
  GTK_LAUNCH_CHECK();
  return GTK_OK;
}

static int raw_attn_entry(const void* q, const void* k, const void* v, const float* bias,
                          const float* mask, float scale, void* out, int64_t B, int64_t H,
                          int64_t N, int64_t D, int dtype, void* ws, size_t ws_bytes,
                          void* stream, int starting) {
  const char* name = starting ? "gtk_triangle_attention_starting" : "gtk_triangle_attention_ending";
  GTK_REQUIRE(dtype == GTK_F32 || dtype == GTK_BF16, GTK_EINVAL, "%s: bad dtype %d", name, dtype);
  GTK_REQUIRE(D == HD, GTK_EUNSUPPORTED, "%s: head dim %lld unsupported (32)", name, (long long)D);
  GTK_REQUIRE(B >= 0 && H >= 1 && N >= 0 && N <= 8192, GTK_EINVAL, "%s: bad shape", name);
  if (B == 0 || N == 0) return GTK_OK;
  GTK_REQUIRE(q && k && v && bias && mask && out && ws, GTK_EINVAL, "%s: null pointer", name);
  const size_t need = gtk_triangle_attention_workspace_size(B, H, N, D, dtype);
  GTK_REQUIRE(ws_bytes >= need, GTK_EWORKSPACE, "%s: workspace %zu < %zu bytes", name, ws_bytes, need);
  hipStream_t st = (hipStream_t)stream;
  if (dtype == GTK_F32) return raw_attention<float>(q, k, v, bias, mask, scale, out, B, H, N, ws, starting, st);
  return raw_attention<bf16>(q, k, v, bias, mask, scale, out, B, H, N, ws, starting, st);
}

// ---------------------------------------------------------------------------
// Fused module forward
// ---------------------------------------------------------------------------
template <typename T>
static int pack_triattn(const gtk_tri_attn_weights* w, int cin, int ch, int H, void* packed,
                        hipStream_t st) {
  PackScope batch(st);  // the packing launches issued as 3
  Carve cv(packed, SIZE_MAX);
  TriAttnPacked<T> p = carve_triattn<T>(cv, cin, ch, H);
  const int wd = w->dtype;
  const int d = ch / H;           // channels of a head
  const int chp = H * HD;         // padded to HD per head
  Pad heads;
  heads.gp = HD;
  heads.g = d;
  const float qscale = kLog2e / sqrtf((float)d);
  int rc;
  if ((rc = launch_to_f32(p.ln_w, w->ln_w, wd, cin, 1.f, 1.f, st))) return rc;
  if ((rc = launch_to_f32(p.ln_b, w->ln_b, wd, cin, 1.f, 0.f, st))) return rc;
  // nn.Linear weight [out][in]: s_out = in, s_in = 1.  Linears after the LayerNorm.
  struct Lin { T* dst; float* bdst; const void* wsrc; const void* bsrc; int out; float scale; Pad pad; };
  const Lin lins[5] = {{p.w_q, p.b_q, w->q_w, nullptr, chp, qscale, heads},
                       {p.w_k, p.b_k, w->k_w, nullptr, chp, 1.f, heads},
                       {p.w_v, p.b_v, w->v_w, nullptr, chp, 1.f, heads},
                       {p.w_g, p.b_g, w->g_w, w->g_b, chp, -kLog2e, heads},
                       {p.w_b, p.b_b, w->tri_w, nullptr, H, kLog2e, Pad()}};
  for (const Lin& l : lins) {
    if ((rc = launch_pack<T>(l.dst, l.wsrc, wd, l.out, cin, cin, 1, l.scale, st, p.ln_w, l.pad))) return rc;
    if ((rc = launch_fold_bias(l.bdst, l.wsrc, l.bsrc, wd, p.ln_b, l.out, cin, cin, 1, l.scale, st, l.pad)))
      return rc;
  }
  // output projection acts on the gated attention output (no LayerNorm);
  // its input channels are the padded heads
  if ((rc = launch_pack<T>(p.w_o, w->o_w, wd, cin, chp, ch, 1, 1.f, st, nullptr, Pad(), heads))) return rc;
  if ((rc = launch_to_f32(p.b_o, w->o_b, wd, cin, 1.f, 0.f, st))) return rc;
  return batch.flush();
}

// chunk_rows > 0: attention rows in chunks of that many rows.
// The triangle bias needs every pair, so it is computed first over all rows;
// then q, k, v^T and the gate of one chunk of rows are computed and attended
// before the next chunk, in a workspace of chunk_rows rows.  Each row's
// attention reads only its own q, k, v^T and gate rows, so the result is the
// same as without chunks.
template <typename T, int CIN, int H>
static int fwd_triattn(const void* x, const float* mask, void* out, const void* packed, int64_t B,
                       int64_t N, int starting, int residual, float eps, float inf, int64_t chunk_rows,
                       void* ws, hipStream_t st) {
  constexpr int CH = H * HD;  // padded heads
  constexpr bool kFast = sizeof(T) == 2 && CIN == 128 && H == 4;
  Carve pc((void*)packed, SIZE_MAX);
  TriAttnPacked<T> w = carve_triattn<T>(pc, CIN, CH, H);
  const int Np = (int)attn_pad(N);
  const bool chunked = chunk_rows > 0 && chunk_rows < N;
  Carve cv(ws, SIZE_MAX);
  AttnWs<T> a = carve_attn_ws<T>(cv, B, Np, H, CH, chunked ? chunk_rows : 0, kFast);
  const int64_t blocks = B * N * ((N + 31) / 32);
  GTK_REQUIRE(blocks < (1ll << 31), GTK_EUNSUPPORTED, "attention grid too large");
  if constexpr (kFast) {
    constexpr int QT = 2;  // two 8-wave blocks of 64 queries per CU (Np > kFlashRhMaxNp)
    const bool rh = Np <= kFlashRhMaxNp;  // (row, head) flash path, fragment-order bf16 bias
    auto prologue = [&](auto mode, int r0, int nrows) {
      constexpr int MODE = decltype(mode)::value;
      const int64_t ptiles = B * (int64_t)nrows * (Np / 32);
      const int grid = (int)std::min<int64_t>(device_cus(), (ptiles + 7) / 8);
      StageTimer timer("triattn_prologue", st);
      triattn_prologue_bf16_kernel<CIN, H, MODE><<<grid, 1024, 0, st>>>(
          (const bf16*)x, mask, w, a, (int)N, Np, starting, eps, ptiles, r0, nrows);
    };
    auto flash = [&](int r0, int nrows) {
      if (rh) {
        // (row, head) blocks, then the output projection
        const int64_t fblocks = B * nrows * H;
        {
          StageTimer timer("triattn_flash", st);
          if (Np <= 256)
            triattn_flash_rh_kernel<256, 8><<<(unsigned)fblocks, 512, 0, st>>>(mask, a, (int)N, Np, starting, r0, nrows, inf);
          else if (Np <= 512)
            triattn_flash_rh_kernel<512, 8><<<(unsigned)fblocks, 512, 0, st>>>(mask, a, (int)N, Np, starting, r0, nrows, inf);
          else
            triattn_flash_rh_kernel<1024, 16><<<(unsigned)fblocks, 1024, 0, st>>>(mask, a, (int)N, Np, starting, r0, nrows, inf);
        }
        GTK_HIP_CHECK(hipGetLastError());
        const int64_t otiles = B * nrows * ((N + 31) / 32);
        const int grid = (int)std::min<int64_t>(2 * device_cus(), (otiles + 7) / 8);
        StageTimer timer("triattn_out", st);
        triattn_out_kernel<CIN><<<grid, 512, 0, st>>>((const bf16*)x, (bf16*)out, w, a, (int)N, Np, starting,
                                                      residual, r0, nrows, otiles);
        return GTK_OK;
      }
      const int64_t fblocks = B * nrows * ((N + 32 * QT - 1) / (32 * QT));
      StageTimer timer("triattn_flash", st);
      triattn_flash_kernel<CIN, H, QT><<<(unsigned)fblocks, 64 * H * QT, 0, st>>>(
          (const bf16*)x, mask, (bf16*)out, w, a, (int)N, Np, starting, residual, r0, nrows, inf);
      return GTK_OK;
    };
    if (!chunked) {
      // every row, padding included
      if (rh) prologue(std::integral_constant<int, 15>(), 0, Np);
      else prologue(std::integral_constant<int, 3>(), 0, Np);
      GTK_LAUNCH_CHECK();
      if (int rc = flash(0, (int)N)) return rc;
      GTK_LAUNCH_CHECK();
    } else {
      // the bias over every row (padding rows and columns are written as zero)
      if (rh) prologue(std::integral_constant<int, 6>(), 0, Np);
      else prologue(std::integral_constant<int, 2>(), 0, Np);
      GTK_LAUNCH_CHECK();
      for (int64_t r0 = 0; r0 < N; r0 += chunk_rows) {
        const int nrows = (int)std::min<int64_t>(chunk_rows, N - r0);
        a.r0 = (int)r0;
        if (rh) prologue(std::integral_constant<int, 9>(), (int)r0, nrows);
        else prologue(std::integral_constant<int, 1>(), (int)r0, nrows);
        GTK_LAUNCH_CHECK();
        if (int rc = flash((int)r0, nrows)) return rc;
        GTK_LAUNCH_CHECK();
      }
    }
  } else {
    auto prologue = [&](int r0, int nrows, int mode) {
      const int64_t ptiles = B * (int64_t)nrows * (Np / 32);
      StageTimer timer("triattn_prologue", st);
      triattn_prologue_kernel<T, CIN, H><<<(unsigned)((ptiles + 3) / 4), 256, 0, st>>>(
          (const T*)x, w, a, (int)B, (int)N, Np, starting, eps, r0, nrows, mode);
    };
    auto attend = [&](int r0, int nrows) {
      const int64_t ablocks = B * nrows * ((N + 31) / 32);
      StageTimer timer("triattn_flash", st);
      triattn_fused_kernel<T, CIN, H><<<(unsigned)ablocks, 64 * H, 0, st>>>(
          (const T*)x, mask, (T*)out, w, a, (int)B, (int)N, Np, starting, residual, inf, r0, nrows);
    };
    if (!chunked) {
      prologue(0, Np, 3);  // every row, padding included
      GTK_LAUNCH_CHECK();
      attend(0, (int)N);
      GTK_LAUNCH_CHECK();
    } else {
      prologue(0, Np, 2);  // the bias over every row
      GTK_LAUNCH_CHECK();
      for (int64_t r0 = 0; r0 < N; r0 += chunk_rows) {
        const int nrows = (int)std::min<int64_t>(chunk_rows, N - r0);
        a.r0 = (int)r0;
        prologue((int)r0, nrows, 1);
        GTK_LAUNCH_CHECK();
        attend((int)r0, nrows);
        GTK_LAUNCH_CHECK();
      }
    }
  }
  return GTK_OK;
}

// c_in in {32, 64, 128}, H in {1, 2, 4}, d = c_h / H in [1, 32] (heads are
// padded to 32 channels); the bf16 kernels built for the module's headline
// shape (c_in = 128, H = 4) run every d, the others run the generic kernels.
static bool triattn_shape_ok(int64_t cin, int64_t ch, int64_t H) {
  return (cin == 32 || cin == 64 || cin == 128) && (H == 1 || H == 2 || H == 4) && ch >= H &&
         ch % H == 0 && ch / H <= HD;
}
static bool triattn_fast_shape(int64_t cin, int64_t H) { return cin == 128 && H == 4; }

template <typename T>
static int fwd_triattn_any(int64_t cin, int64_t H, const void* x, const float* mask, void* out,
                           const void* packed, int64_t B, int64_t N, int starting, int residual,
                           float eps, float inf, int64_t chunk_rows, void* ws, hipStream_t st) {
#define GTK_TA(C, HH)                                                                               \
  if (cin == C && H == HH)                                                                       \
    return fwd_triattn<T, C, HH>(x, mask, out, packed, B, N, starting, residual, eps, inf, chunk_rows, \
                                 ws, st);
  GTK_TA(128, 4) GTK_TA(128, 2) GTK_TA(128, 1)
  GTK_TA(64, 4) GTK_TA(64, 2) GTK_TA(64, 1)
  GTK_TA(32, 4) GTK_TA(32, 2) GTK_TA(32, 1)
#undef GTK_TA
  set_error("tri_attn: c_in=%lld H=%lld unsupported", (long long)cin, (long long)H);
  return GTK_EUNSUPPORTED;
}

}  // namespace gtk

using namespace gtk;

extern "C" size_t gtk_triangle_attention_workspace_size(int64_t B, int64_t H, int64_t N, int64_t D,
                                                        int dtype) {
  if (B < 0 || H < 1 || N < 0 || D != HD) return 0;
  Carve cv(nullptr, SIZE_MAX);
  if (dtype == GTK_F32) carve_attn_ws<float>(cv, B, attn_pad(N), (int)H, 0);
  else carve_attn_ws<bf16>(cv, B, attn_pad(N), (int)H, 0);
  return cv.off;
}

extern "C" int gtk_triangle_attention_starting(const void* q, const void* k, const void* v,
                                               const float* bias, const float* mask, float scale,
                                               void* out, int64_t B, int64_t H, int64_t N,
                                               int64_t D, int dtype, void* ws, size_t ws_bytes,
                                               void* stream) {
  return raw_attn_entry(q, k, v, bias, mask, scale, out, B, H, N, D, dtype, ws, ws_bytes, stream, 1);
}

extern "C" int gtk_triangle_attention_ending(const void* q, const void* k, const void* v,
                                             const float* bias, const float* mask, float scale,
                                             void* out, int64_t B, int64_t H, int64_t N, int64_t D,
                                             int dtype, void* ws, size_t ws_bytes, void* stream) {
  return raw_attn_entry(q, k, v, bias, mask, scale, out, B, H, N, D, dtype, ws, ws_bytes, stream, 0);
}

extern "C" size_t gtk_tri_attn_packed_size(int64_t c_in, int64_t c_h, int64_t H, int dtype) {
  if (!triattn_shape_ok(c_in, c_h, H)) return 0;
  Carve cv(nullptr, SIZE_MAX);
  if (dtype == GTK_F32) carve_triattn<float>(cv, (int)c_in, (int)c_h, (int)H);
  else carve_triattn<bf16>(cv, (int)c_in, (int)c_h, (int)H);
  return cv.off;
}

extern "C" int gtk_tri_attn_pack(const gtk_tri_attn_weights* w, int64_t c_in, int64_t c_h,
                                 int64_t H, int dtype, void* packed, size_t packed_bytes,
                                 void* stream) {
  GTK_REQUIRE(w && packed, GTK_EINVAL, "gtk_tri_attn_pack: null pointer");
  GTK_REQUIRE(dtype == GTK_F32 || dtype == GTK_BF16, GTK_EINVAL, "gtk_tri_attn_pack: bad dtype %d", dtype);
  GTK_REQUIRE(w->dtype == GTK_F32 || w->dtype == GTK_BF16, GTK_EINVAL,
              "gtk_tri_attn_pack: bad weight dtype %d", w->dtype);
  GTK_REQUIRE(triattn_shape_ok(c_in, c_h, H), GTK_EUNSUPPORTED,
              "gtk_tri_attn_pack: c_in=%lld c_h=%lld H=%lld unsupported (c_in in {32,64,128}, H in "
              "{1,2,4}, c_h / H <= 32)",
              (long long)c_in, (long long)c_h, (long long)H);
  GTK_REQUIRE(w->q_w && w->k_w && w->v_w && w->g_w && w->o_w && w->tri_w, GTK_EINVAL,
              "gtk_tri_attn_pack: null weight");
  const size_t need = gtk_tri_attn_packed_size(c_in, c_h, H, dtype);
  GTK_REQUIRE(packed_bytes >= need, GTK_EWORKSPACE, "gtk_tri_attn_pack: buffer %zu < %zu bytes",
              packed_bytes, need);
  hipStream_t st = (hipStream_t)stream;
  if (dtype == GTK_F32) return pack_triattn<float>(w, (int)c_in, (int)c_h, (int)H, packed, st);
  return pack_triattn<bf16>(w, (int)c_in, (int)c_h, (int)H, packed, st);
}

extern "C" size_t gtk_tri_attn_workspace_size_chunked(int64_t B, int64_t N, int64_t c_in,
                                                      int64_t c_h, int64_t H, int64_t chunk_rows,
                                                      int dtype) {
  if (!triattn_shape_ok(c_in, c_h, H) || B < 0 || N < 0 || chunk_rows < 0) return 0;
  if (dtype != GTK_F32 && dtype != GTK_BF16) return 0;
  const bool fast = dtype == GTK_BF16 && triattn_fast_shape(c_in, H);
  Carve cv(nullptr, SIZE_MAX);
  const int64_t rows = chunk_rows > 0 && chunk_rows < N ? chunk_rows : 0;
  const int chp = (int)H * HD;
  if (dtype == GTK_F32) carve_attn_ws<float>(cv, B, attn_pad(N), (int)H, chp, rows, false);
  else carve_attn_ws<bf16>(cv, B, attn_pad(N), (int)H, chp, rows, fast);
  return cv.off;
}

extern "C" size_t gtk_tri_attn_workspace_size(int64_t B, int64_t N, int64_t c_in, int64_t c_h,
                                              int64_t H, int dtype) {
  return gtk_tri_attn_workspace_size_chunked(B, N, c_in, c_h, H, 0, dtype);
}

extern "C" int gtk_tri_attn_forward_chunked(const void* x, const float* mask, void* out,
                                            const void* packed, int64_t B, int64_t N, int64_t c_in,
                                            int64_t c_h, int64_t H, int starting, int residual,
                                            float eps, float inf, int64_t chunk_rows, int dtype,
                                            void* ws, size_t ws_bytes, void* stream) {
  GTK_REQUIRE(dtype == GTK_F32 || dtype == GTK_BF16, GTK_EINVAL, "gtk_tri_attn_forward: bad dtype %d", dtype);
  GTK_REQUIRE(triattn_shape_ok(c_in, c_h, H), GTK_EUNSUPPORTED,
              "gtk_tri_attn_forward: c_in=%lld c_h=%lld H=%lld unsupported (c_in in {32,64,128}, "
              "H in {1,2,4}, c_h / H <= 32)",
              (long long)c_in, (long long)c_h, (long long)H);
  GTK_REQUIRE(B >= 0 && N >= 0 && N <= 8192 && chunk_rows >= 0, GTK_EINVAL,
              "gtk_tri_attn_forward: bad shape");
  GTK_REQUIRE(abs_at_most(inf, 1e37f), GTK_EINVAL,
              "gtk_tri_attn_forward: |inf| must be at most 1e37, got %g", (double)inf);
  if (B == 0 || N == 0) return GTK_OK;
  GTK_REQUIRE(x && out && packed && ws, GTK_EINVAL, "gtk_tri_attn_forward: null pointer");
  const size_t need = gtk_tri_attn_workspace_size_chunked(B, N, c_in, c_h, H, chunk_rows, dtype);
  GTK_REQUIRE(ws_bytes >= need, GTK_EWORKSPACE, "gtk_tri_attn_forward: workspace %zu < %zu bytes",
              ws_bytes, need);
  hipStream_t st = (hipStream_t)stream;
  if (dtype == GTK_F32)
    return fwd_triattn_any<float>(c_in, H, x, mask, out, packed, B, N, starting, residual, eps, inf,
                                  chunk_rows, ws, st);
  return fwd_triattn_any<bf16>(c_in, H, x, mask, out, packed, B, N, starting, residual, eps, inf,
                               chunk_rows, ws, st);
}

extern "C" int gtk_tri_attn_forward(const void* x, const float* mask, void* out, const void* packed,
                                    int64_t B, int64_t N, int64_t c_in, int64_t c_h, int64_t H,
                                    int starting, int residual, float eps, float inf, int dtype,
                                    void* ws, size_t ws_bytes, void* stream) {
  return gtk_tri_attn_forward_chunked(x, mask, out, packed, B, N, c_in, c_h, H, starting, residual,
                                      eps, inf, 0, dtype, ws, ws_bytes, stream);
}
