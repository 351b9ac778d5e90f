// Triangle multiplicative update (outgoing / incoming) for gfx950.
//
// Three kernels, all reading/writing HBM in the layouts below:
//
//  1. prologue   z[B][N][N][c_z]  ->  A, Bm planes [B][c][Np][Np]
//       LN_in in fragment layout, the four c_z->c projections on the matrix
//       cores, sigmoid gates and the pair mask fused; results written
//       channel-major so that the contraction reads both operands with k
//       contiguous.  Outgoing stores pair (p,q) at plane[c][p][q], incoming at
//       plane[c][q][p]; after that both directions are the same GEMM.
//  2. contract   X[b][c] = A[b][c] . Bm[b][c]^T     (B*c GEMMs of Np x Np x Np)
//       128x128 (or 64x64) tiles, 4 waves, k staged through LDS in 128-byte
//       rows with double buffering, fp32 accumulation.
//  3. epilogue   X planes + z  ->  out[B][N][N][c_z]
//       X tile transposed through LDS into fragment layout, LN_out and W_z on
//       the matrix cores, gate sigmoid(LN_in(z) W_g^T + b_g) recomputed from z
//       (cheaper than storing it), optional residual add.
//
// Np = N rounded up to 64; the prologue writes zeros for padded pairs so the
// contraction needs no bounds checks.
#include <algorithm>
#include <type_traits>

#include "capi_util.hpp"
#include "common.hpp"
#include "pack.hpp"
#include "tri_mul_internal.hpp"

namespace gtk {

// Plane stride of the forward's channel planes: rows * Np elements plus 256
// bytes.  A power-of-two stride (2 MiB at N = 1024) sends the 256 plane
// stores of a prologue step to the same HBM channels: 512 MiB of planes
// written in 162 us at N = 1024, against 80 us with the padded stride.
template <typename T>
inline int64_t plane_stride(int64_t rows, int64_t Np) {
  return rows * Np + 256 / (int64_t)sizeof(T);
}

// ---------------------------------------------------------------------------
// 1. Prologue
//    Both prologues write plane rows f = r0 .. r0 + nrows - 1 as rows
//    0 .. nrows - 1 of nrows x Np planes, for sides side_lo .. side_hi - 1
//    (0: A, 1: Bm).  Whole planes: r0 = 0, nrows = Np, sides 0 .. 1; the row
//    chunks of the memory-bounded mode write Bm once over all rows and A one
//    chunk of rows at a time.
// ---------------------------------------------------------------------------
template <typename T, int CZ, int CH>
__global__ __launch_bounds__(256) void trimul_prologue_kernel(
    const T* __restrict__ z, const float* __restrict__ mask, T* __restrict__ pa,
    T* __restrict__ pb, TriMulPacked<T> w, int B, int N, int Np, int outgoing, float eps,
    int r0, int nrows, int side_lo, int side_hi, int64_t plane) {
  const int lane = threadIdx.x & 63;
  const int half = lane >> 5;
  const int t32 = lane & 31;
  const int vtiles = Np / 32;
  const int64_t tile = (int64_t)blockIdx.x * 4 + wave_id();
  if (tile >= (int64_t)B * nrows * vtiles) return;
  const int vt = (int)(tile % vtiles);
  const int fl = (int)((tile / vtiles) % nrows);
  const int f = r0 + fl;
  const int b = (int)(tile / ((int64_t)vtiles * nrows));
  const int v = vt * 32 + t32;
  const int p = outgoing ? f : v;
  const int q = outgoing ? v : f;
  const bool valid = (p < N) && (q < N);
  const int64_t pair = ((int64_t)b * N + (valid ? p : 0)) * N + (valid ? q : 0);

  RowHalf<CZ> rh;
  load_row_half<T, CZ>(rh, z + pair * CZ, valid);
  const f32x2 st = row_stats<CZ>(rh, eps);
  Frag<T> xf[CZ / 16];
  if constexpr (trimul_folded<CZ, CH>()) ln_to_frags<T, CZ>(xf, rh, st);
  else ln_affine_to_frags<T, CZ>(xf, rh, st, w.ln_in_w, w.ln_in_b);
  const float m = valid ? (mask ? mask[pair] : 1.0f) : 0.0f;

  const int64_t off_fv = (int64_t)fl * Np + v;
#pragma unroll 1
  for (int side = side_lo; side < side_hi; ++side) {
    const T* wp = side ? w.w_bp : w.w_ap;
    const T* wg = side ? w.w_bg : w.w_ag;
    const float* bp = side ? w.b_bp : w.b_ap;
    const float* bg = side ? w.b_bg : w.b_ag;
    T* dst = (side ? pb : pa) + (int64_t)b * CH * plane + off_fv;
#pragma unroll 1
    for (int nt = 0; nt < CH / 32; ++nt) {
      const f32x16 ap = row_gemm_tile<T, CZ, true>(xf, wp, nt);
      const f32x16 ag = row_gemm_tile<T, CZ, true>(xf, wg, nt);
#pragma unroll
      for (int g = 0; g < 4; ++g) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int c = nt * 32 + 8 * g + 4 * half + r;
          const float val = (ap[4 * g + r] + bp[c]) * gate_from_u(ag[4 * g + r] + bg[c]) * m;
          dst[(int64_t)c * plane] = cvt<T>(val);
        }
      }
    }
  }
}

// ---------------------------------------------------------------------------
// 1b. bf16 prologue: persistent, 8 waves per CU (256 VGPRs each) with the
//     four packed c_z->c weights resident in LDS (4 x 32 KiB, loaded with
//     direct global->LDS copies).  Each wave step covers two 32-pair tiles of
//     one row: every weight fragment read from LDS feeds both tiles' MFMAs,
//     halving LDS traffic per MFMA.
//
//     The pairs are the MFMA A operand (rows) and the weights the B operand
//     (columns = channels).  A-operand row i carries tile pair
//     16*((i>>2)&1) + 4*(i>>3) + (i&3), which makes accumulator register j of
//     lane l hold pair 16*(l>>5) + j of channel (l&31): every lane ends with 16
//     consecutive pairs of one channel and writes them as two 16-byte stores.
//     The gate bias enters as a factor, 2^(u+b) = 2^u * 2^b, so the gate costs
//     one FMA beside its two transcendental instructions.
//     Each 32-channel tile of the result goes out through the wave's LDS
//     staging rows, 16 channels at a time (the lanes of those channels write
//     their 2 x 32 bytes, then every lane stores 16 bytes of one channel's
//     128-byte row): each store instruction writes 8 whole cache lines
//     instead of 32 lines in two 16-byte pieces each (59.6 -> 58.7 us at
//     N = 512, bit-identical).  The z rows load without a branch: an
//     invalid pair reads pair (b, 0, 0) and its mask of 0 zeroes its output.
//     TPS = 1 (one tile a step) when two-tile steps would leave waves of the
//     grid without work (N = 256: 1024 steps for 2048 waves; 23.6 -> 19.5 us,
//     bit-identical): then each weight fragment feeds one tile's products.
//     FP8 (the fp8 a/b storage experiment): the planes hold OCP fp8 E4M3
//     values (v_cvt_pk_fp8_f32, round to nearest even; clamped to +-448
//     first), one 16-byte store per lane and channel tile.
// ---------------------------------------------------------------------------
template <int CZ, int CH, bool FP8 = false, bool RANGE = false, int TPS = 2>
__global__ __launch_bounds__(512) void trimul_prologue_bf16_kernel(
    const bf16* __restrict__ z, const float* __restrict__ mask,
    std::conditional_t<FP8, uint8_t, bf16>* __restrict__ pa,
    std::conditional_t<FP8, uint8_t, bf16>* __restrict__ pb, TriMulPacked<bf16> w, int N, int Np,
    int outgoing, float eps, int64_t ntiles, int r0, int nrows, int side_lo, int side_hi,
    int64_t plane) {
  using OutT = std::conditional_t<FP8, uint8_t, bf16>;
  if constexpr (!RANGE) {  // whole planes, both sides: the range is known here
    r0 = 0;
    nrows = Np;
    side_lo = 0;
    side_hi = 2;
  }
  constexpr int WAVES = 8;
  constexpr int KCH = CZ / 16;
  constexpr int PE = (CH / 32) * KCH * 512;  // packed elements of one projection
  __shared__ __attribute__((aligned(1024))) bf16 wl[4][PE];
  // biases in LDS: read in the loop between stores, a global load would wait
  // for the stores issued before it (loads complete in issue order)
  __shared__ float bl[2][2][CH];  // [side][projection, gate as 2^b_g]
  // the pair mask of each wave's current step (64 consecutive pairs)
  __shared__ __attribute__((aligned(16))) float ml[WAVES][64];
  // output staging: 16 channel rows x 128 bytes (64 pairs), pitch 144
  constexpr int SPITCH = 144;
  __shared__ __attribute__((aligned(16))) char stg[FP8 ? 1 : WAVES][FP8 ? 16 : 16 * SPITCH];
  copy_to_lds_async(wl[0], w.w_ap, PE * 2);
  copy_to_lds_async(wl[1], w.w_ag, PE * 2);
  copy_to_lds_async(wl[2], w.w_bp, PE * 2);
  copy_to_lds_async(wl[3], w.w_bg, PE * 2);
  for (int t = threadIdx.x; t < CH; t += blockDim.x) {
    bl[0][0][t] = w.b_ap[t];
    bl[0][1][t] = fmaxf(__builtin_amdgcn_exp2f(w.b_ag[t]), 1.17549435e-38f);
    bl[1][0][t] = w.b_bp[t];
    bl[1][1][t] = fmaxf(__builtin_amdgcn_exp2f(w.b_bg[t]), 1.17549435e-38f);
  }
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();

  const int lane = threadIdx.x & 63;
  const int wave = wave_id();
  const int half = lane >> 5;
  const int i32 = lane & 31;
  const int prow = 16 * ((i32 >> 2) & 1) + 4 * (i32 >> 3) + (i32 & 3);
  const int vtiles = Np / 32;  // even: Np is a multiple of 64
  const int64_t nsteps = ntiles / TPS;  // ntiles is even (Np / 32 tiles a row)

  // raw z rows of the TPS tiles of step s (zeros outside the N x N pair grid)
  auto load_z = [&](Frag<bf16> (*zr)[KCH], int64_t s) {
    const int64_t tile = (int64_t)TPS * s;
    const int vt = (int)(tile % vtiles);
    const int f = r0 + (int)((tile / vtiles) % nrows);
    const int b = (int)(tile / ((int64_t)vtiles * nrows));
#pragma unroll
    for (int u = 0; u < TPS; ++u) {
      const int v = (vt + u) * 32 + prow;
      const int p = outgoing ? f : v, q = outgoing ? v : f;
      const bool valid = p < N && q < N;
      // an invalid pair reads pair (b, 0, 0): its mask is 0, so its outputs
      // are zero all the same, and the loads need no branch
      const bf16* row = z + (((int64_t)b * N + (valid ? p : 0)) * N + (valid ? q : 0)) * CZ + half * (CZ / 2);
#pragma unroll
      for (int ch = 0; ch < KCH; ++ch) zr[u][ch].load(row + ch * 8);
    }
  };

  // The mask of the step's 64 pairs (zero outside the grid): one load per
  // lane (pair vt*32 + lane), staged in the wave's LDS slot and read back by
  // each lane as its 16 output pairs of a tile when it stores.
  auto load_mask = [&](int64_t s) {
    const int64_t tile = (int64_t)TPS * s;
    const int vt = (int)(tile % vtiles);
    const int f = r0 + (int)((tile / vtiles) % nrows);
    const int b = (int)(tile / ((int64_t)vtiles * nrows));
    const int v = vt * 32 + lane;
    const bool ok = f < N && v < N;
    const int64_t idx = ((int64_t)b * N + (outgoing ? f : v)) * N + (outgoing ? v : f);
    return ok ? (mask ? mask[ok ? idx : 0] : 1.f) : 0.f;
  };

  // steps dealt round-robin over the blocks first, so a small problem still
  // reaches every CU (a block may then run fewer than WAVES busy waves)
  int64_t s = (int64_t)wave * gridDim.x + blockIdx.x;
  const int64_t sstride = (int64_t)gridDim.x * WAVES;
  // this wave's first step: rows and mask in flight (the next step's are
  // loaded ahead of each step's stores)
  Frag<bf16> zr[TPS][KCH];
  float mv = 0.f;
  if (s < nsteps) {
    load_z(zr, s);
    mv = load_mask(s);
  }
  for (; s < nsteps; s += sstride) {
    const int64_t tile = (int64_t)TPS * s;
    const int vt = (int)(tile % vtiles);
    const int fl = (int)((tile / vtiles) % nrows);  // row of the written planes
    const int b = (int)(tile / ((int64_t)vtiles * nrows));
    Frag<bf16> xf[TPS][KCH];
#pragma unroll
    for (int u = 0; u < TPS; ++u) ln_frags_bf16<CZ>(xf[u], zr[u], eps);
    ml[wave][lane] = mv;
    if (s + sstride < nsteps) {
      load_z(zr, s + sstride);
      mv = load_mask(s + sstride);
    }
#pragma unroll 1
    for (int side = side_lo; side < side_hi; ++side) {
      const bf16* wp = wl[2 * side];
      const bf16* wg = wl[2 * side + 1];
      const float* bp = bl[side][0];
      const float* ebgs = bl[side][1];
      OutT* dst = (side ? pb : pa) + (int64_t)b * CH * plane + (int64_t)fl * Np + vt * 32 + 16 * half;
#pragma unroll 1
      for (int ct = 0; ct < CH / 32; ++ct) {
        Frag<bf16> wfp, wfg;
        load_wfrag_lds(wfp, wp, ct, 0, KCH);
        load_wfrag_lds(wfg, wg, ct, 0, KCH);
        f32x16 apv[TPS], agv[TPS];
#pragma unroll
        for (int u = 0; u < TPS; ++u) {
          apv[u] = mma0(xf[u][0], wfp);
          agv[u] = mma0(xf[u][0], wfg);
        }
#pragma unroll
        for (int ks = 1; ks < KCH; ++ks) {
          load_wfrag_lds(wfp, wp, ct, ks, KCH);
          load_wfrag_lds(wfg, wg, ct, ks, KCH);
#pragma unroll
          for (int u = 0; u < TPS; ++u) {
            mma(apv[u], xf[u][ks], wfp);
            mma(agv[u], xf[u][ks], wfg);
          }
        }
        const int cc = ct * 32 + i32;
        const float bpc = bp[cc];
        const float ebg = ebgs[cc];
        uint32_t pku[TPS][8];
#pragma unroll
        for (int u = 0; u < TPS; ++u) {
          const f32x16& ap = apv[u];
          const f32x16& ag = agv[u];
          // mask of this lane's pairs 32u + 16*half .. +15
          float mk[16];
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            const f32x4 m4 = *reinterpret_cast<const f32x4*>(&ml[wave][32 * u + 16 * half + 4 * q]);
#pragma unroll
            for (int e = 0; e < 4; ++e) mk[4 * q + e] = m4[e];
          }
          uint32_t pk[8] = {};
#pragma unroll
          for (int j = 0; j < 16; j += 2) {
            const float o0 = (ap[j] + bpc) *
                             __builtin_amdgcn_rcpf(fmaf(__builtin_amdgcn_exp2f(ag[j]), ebg, 1.f)) * mk[j];
            const float o1 = (ap[j + 1] + bpc) *
                             __builtin_amdgcn_rcpf(fmaf(__builtin_amdgcn_exp2f(ag[j + 1]), ebg, 1.f)) *
                             mk[j + 1];
            if constexpr (FP8) {
              const float c0 = __builtin_amdgcn_fmed3f(o0, -448.f, 448.f);
              const float c1 = __builtin_amdgcn_fmed3f(o1, -448.f, 448.f);
              // pairs j, j+1 -> bytes (j & 3), (j & 3) + 1 of dword j / 4
              if ((j & 2) == 0)
                pk[j / 4] = (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(c0, c1, (int)pk[j / 4], false);
              else
                pk[j / 4] = (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(c0, c1, (int)pk[j / 4], true);
            } else {
              pk[j / 2] = pack_bf16x2(o0, o1);
            }
          }
          if constexpr (FP8) {
            uint4* o = reinterpret_cast<uint4*>(dst + (int64_t)cc * plane + 32 * u);
            o[0] = make_uint4(pk[0], pk[1], pk[2], pk[3]);
          } else {
#pragma unroll
            for (int e = 0; e < 8; ++e) pku[u][e] = pk[e];
          }
        }
        if constexpr (!FP8) {
          // Through the wave's staging rows, 16 channels at a time: lanes of
          // channels 16h' .. 16h'+15 write their 2 x 32 bytes, then every
          // lane stores 16 bytes of one channel's 128-byte row, so each store
          // instruction covers 8 whole cache lines.
          char* const sw = stg[wave];
          OutT* const row0 = dst - 16 * half;  // pair vt*32 of plane 0, row fl
#pragma unroll
          for (int hp = 0; hp < 2; ++hp) {
            if ((i32 >> 4) == hp) {
              char* wr = sw + (i32 & 15) * SPITCH + 32 * half;
#pragma unroll
              for (int u = 0; u < TPS; ++u) {
                *reinterpret_cast<uint4*>(wr + 64 * u) =
                    make_uint4(pku[u][0], pku[u][1], pku[u][2], pku[u][3]);
                *reinterpret_cast<uint4*>(wr + 64 * u + 16) =
                    make_uint4(pku[u][4], pku[u][5], pku[u][6], pku[u][7]);
              }
            }
            __builtin_amdgcn_wave_barrier();
            // rows of 64 * TPS bytes: LPR lanes a row, 16 / TPS rows an instruction
            constexpr int LPR = 4 * TPS;
#pragma unroll
            for (int m = 0; m < TPS; ++m) {
              const int r = lane / LPR + (16 / TPS) * m;
              const int c16 = lane % LPR;
              const uint4 v = *reinterpret_cast<const uint4*>(sw + r * SPITCH + c16 * 16);
              *reinterpret_cast<uint4*>(row0 + (int64_t)(ct * 32 + 16 * hp + r) * plane + c16 * 8) = v;
            }
            __builtin_amdgcn_wave_barrier();
          }
        }
      }
    }
  }
}

// ---------------------------------------------------------------------------
// 2. Per-channel contraction  X = A . Bm^T   (Bm: [Np][Np] planes; A, X:
//    [Mi][Np], Mi = Np for whole planes, fewer rows for a row chunk)
// ---------------------------------------------------------------------------
template <typename T, int TILE>
__global__ __launch_bounds__(256) void trimul_contract_kernel(const T* __restrict__ pa,
                                                              const T* __restrict__ pb,
                                                              T* __restrict__ px, int Np, int Mi,
                                                              int64_t nplanes, int64_t plane,
                                                              int64_t plane_ax) {
  constexpr int BK = 128 / sizeof(T);            // k elements per stage (128-byte rows)
  constexpr int PITCH = 144;                     // LDS row pitch in bytes (16 B pad)
  constexpr int WT = TILE / 2;                   // per-wave tile (2x2 waves)
  constexpr int MB = WT / 32;                    // 32x32 MFMA blocks per wave side
  constexpr int CHUNKS = TILE * 8;               // 16-byte chunks per operand per stage
  constexpr int CPT = CHUNKS / 256;              // chunks per thread per operand
  constexpr int EPC = 16 / sizeof(T);            // elements per 16-byte chunk
  __shared__ __attribute__((aligned(16))) char smem[2][2][TILE * PITCH];

  const int ti_n = Mi / TILE, tj_n = Np / TILE;
  const int64_t total = (int64_t)ti_n * tj_n * nplanes;
  const int64_t lin = xcd_remap((int64_t)blockIdx.x, total);
  const int64_t pl = lin / ((int64_t)ti_n * tj_n);
  const int trem = (int)(lin % ((int64_t)ti_n * tj_n));
  const int i0 = (trem / tj_n) * TILE;
  const int j0 = (trem % tj_n) * TILE;
  // plane strides: Bm (Np x Np rows), A and X (Mi x Np rows)
  const T* A = pa + pl * plane_ax;
  const T* Bm = pb + pl * plane;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wi = (wave >> 1) * WT;  // wave row offset (i)
  const int wj = (wave & 1) * WT;   // wave col offset (j)

  f32x16 acc[MB][MB];
#pragma unroll
  for (int x = 0; x < MB; ++x)
#pragma unroll
    for (int y = 0; y < MB; ++y) acc[x][y] = zero16();

  f32x4 ra[CPT], rb[CPT];
  auto gload = [&](int k0) {
#pragma unroll
    for (int u = 0; u < CPT; ++u) {
      const int id = tid + 256 * u;
      const int row = id >> 3, cc = id & 7;
      ra[u] = *reinterpret_cast<const f32x4*>(A + (int64_t)(i0 + row) * Np + k0 + cc * EPC);
      rb[u] = *reinterpret_cast<const f32x4*>(Bm + (int64_t)(j0 + row) * Np + k0 + cc * EPC);
    }
  };
  auto sstore = [&](int buf) {
#pragma unroll
    for (int u = 0; u < CPT; ++u) {
      const int id = tid + 256 * u;
      const int row = id >> 3, cc = id & 7;
      *reinterpret_cast<f32x4*>(&smem[buf][0][row * PITCH + cc * 16]) = ra[u];
      *reinterpret_cast<f32x4*>(&smem[buf][1][row * PITCH + cc * 16]) = rb[u];
    }
  };

  const int KT = Np / BK;
  gload(0);
  sstore(0);
  __syncthreads();
  const int half = lane >> 5;
  for (int kt = 0; kt < KT; ++kt) {
    const int cur = kt & 1;
    if (kt + 1 < KT) gload((kt + 1) * BK);
#pragma unroll
    for (int kc = 0; kc < BK / 16; ++kc) {
      Frag<T> fa[MB], fb[MB];
#pragma unroll
      for (int x = 0; x < MB; ++x) {
        const int ra_row = wi + x * 32 + (lane & 31);
        const int rb_row = wj + x * 32 + (lane & 31);
        const int koff = (kc * 16 + half * 8) * (int)sizeof(T);
        fa[x].load(reinterpret_cast<const T*>(&smem[cur][0][ra_row * PITCH + koff]));
        fb[x].load(reinterpret_cast<const T*>(&smem[cur][1][rb_row * PITCH + koff]));
      }
#pragma unroll
      for (int x = 0; x < MB; ++x)
#pragma unroll
        for (int y = 0; y < MB; ++y) mma(acc[x][y], fb[y], fa[x]);  // rows j, cols i
    }
    if (kt + 1 < KT) sstore(cur ^ 1);
    __syncthreads();
  }

  // acc[x][y]: lane holds X[i = wi + 32x + (l&31)][j = wj + 32y + 8g + 4h + r]
  T* X = px + pl * plane_ax;
#pragma unroll
  for (int x = 0; x < MB; ++x) {
    const int i = i0 + wi + x * 32 + (lane & 31);
#pragma unroll
    for (int y = 0; y < MB; ++y) {
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int j = j0 + wj + y * 32 + 8 * g + 4 * half;
        store4(X + (int64_t)i * Np + j, acc[x][y][4 * g + 0], acc[x][y][4 * g + 1],
               acc[x][y][4 * g + 2], acc[x][y][4 * g + 3]);
      }
    }
  }
}

// ---------------------------------------------------------------------------
// 2b. bf16 contraction: TI x TJ output tiles, blocks of (TI/64)x(TJ/64)
//     waves, each wave 64x64.  k advances in stages of 64: the A and Bm
//     panels (TI and TJ rows x 128 bytes, whole cache lines) move by direct
//     global->LDS copies into a double buffer, the next stage issued before
//     the current one is consumed, so no VGPRs stage the operands.  The
//     panels are re-read once per tile of the other operand, so the 256x256
//     tile halves the L2->LDS traffic of a 128x128 one.  Panel rows are
//     chunk-swizzled (16-byte chunk c of row r sits at c ^ f(r)), which makes
//     the fragment reads bank-conflict free.
//     Persistent: block b walks tiles b, b + gridDim.x, ... (gridDim.x a
//     multiple of 8, so the XCD-aware order holds for every step).  At the
//     last k stage the next tile's first stage is issued into the stage just
//     freed, and the finished tile is stored from the accumulators while that
//     copy is in flight (one block per CU at 256x256: its stores would
//     otherwise overlap no copy or MFMA; 48.4 -> 44.5 us at N = 512).
//   * LT / RT: the operand is given transposed, as the plane L^T [k][i]
//     (R^T [k][j]) of whole Np x Np planes, which is how the backward's
//     dA = dX Bm and dB = dX^T A read the forward planes without transposing
//     them first.  Such a panel sits in LDS as 64 k rows of TI (TJ) columns,
//     16-byte chunk c of row r at c ^ 4(r % 4), and its fragments (8
//     consecutive k of one column a lane) come from two transposing reads
//     (ds_read_b64_tr_b16): within 16 lanes, lane L takes element L % 4 of
//     the pieces at the addresses of lanes L/4, 4 + L/4, 8 + L/4 and
//     12 + L/4, so with supplier lane s at row k0 + s/4, columns cb + 4(s%4)
//     .. +3, lane L receives rows k0 .. k0 + 3 of column cb + L.  The 32
//     lanes served together read four rows at four chunks each, which the
//     swizzle places in 16 distinct chunks of a 256-byte bank window (with
//     c ^ 2(r % 4) the two 16-lane halves collided: 4 conflict cycles a
//     read in the counters).  Products, sums and their order are those of
//     the plain form on the transposed planes.
// ---------------------------------------------------------------------------
template <int TI, int TJ, bool LT = false, bool RT = false>
__global__ __launch_bounds__(64 * (TI / 64) * (TJ / 64)) void trimul_contract_bf16_kernel(
    const bf16* __restrict__ pa, const bf16* __restrict__ pb, bf16* __restrict__ px, int Np,
    int Mi, int64_t nplanes, int64_t plane, int64_t plane_ax) {
  constexpr int BK = 64, NS = 2;
  constexpr int NW = (TI / 64) * (TJ / 64);         // waves
  constexpr int RPR = 1024 / (2 * BK);              // panel rows per 1 KiB copy
  constexpr int CPR = BK / 8;                       // 16-byte chunks per panel row
  static_assert((TI / RPR) % NW == 0 && (TJ / RPR) % NW == 0, "copies split evenly");
  // transposed panels: 64 rows of TI (TJ) columns, 1 KiB copies of RPT rows
  constexpr int RPTA = 512 / TI, CPTA = TI / 8, RPTB = 512 / TJ, CPTB = TJ / 8;
  static_assert((BK / RPTA) == TI / RPR && (BK / RPTB) == TJ / RPR, "same copy count either way");
  auto tswz = [](int r) { return 4 * (r & 3); };
  __shared__ __attribute__((aligned(1024))) bf16 ring[NS * (TI + TJ) * BK];

  const int ti_n = Mi / TI, tj_n = Np / TJ;
  const int64_t total = (int64_t)ti_n * tj_n * nplanes;
  // plane strides: Bm (Np x Np rows), A and X (Mi x Np rows)

  const int lane = threadIdx.x & 63;
  const int wave = wave_id();
  const int half = lane >> 5;
  const int wi = (wave / (TJ / 64)) * 64;  // wave row offset (i)
  const int wj = (wave % (TJ / 64)) * 64;  // wave col offset (j)
  // chunk swizzle of panel row r: distinct for any rows that share LDS banks,
  // whether 8 or 16 lanes are served per cycle
  auto pswz = [](int r) { return (r ^ (r >> 3)) & 7; };

  // copies: a panel is (rows/RPR) regions of RPR rows x CPR chunks; wave w
  // moves regions w, w+NW, ... of both panels; lane l lands at row
  // RPR*n + l/CPR, chunk l%CPR.  The per-lane byte offsets inside a panel
  // are the same for every tile; the panel bases are wave-uniform.
  constexpr int RA = TI / RPR / NW, RB = TJ / RPR / NW;
  uint32_t voA[RA], voB[RB];
#pragma unroll
  for (int u = 0; u < RA; ++u) {
    if constexpr (LT) {
      const int row = RPTA * (wave + u * NW) + lane / CPTA;  // k row
      voA[u] = (uint32_t)((row * Np + 8 * ((lane % CPTA) ^ tswz(row))) * 2);
    } else {
      const int row = RPR * (wave + u * NW) + lane / CPR;
      voA[u] = (uint32_t)((row * Np + 8 * ((lane % CPR) ^ pswz(row))) * 2);
    }
  }
#pragma unroll
  for (int u = 0; u < RB; ++u) {
    if constexpr (RT) {
      const int row = RPTB * (wave + u * NW) + lane / CPTB;  // k row
      voB[u] = (uint32_t)((row * Np + 8 * ((lane % CPTB) ^ tswz(row))) * 2);
    } else {
      const int row = RPR * (wave + u * NW) + lane / CPR;
      voB[u] = (uint32_t)((row * Np + 8 * ((lane % CPR) ^ pswz(row))) * 2);
    }
  }
  const uint32_t lds_a = lds_addr(ring), lds_b = lds_addr(ring + NS * TI * BK);
  const bf16* Ab = nullptr;  // panel bases of the tile being loaded
  const bf16* Bb = nullptr;
  bf16* X = nullptr;         // its output tile
  auto setup = [&](int64_t v) {
    const int64_t lin = xcd_remap(v, total);
    const int64_t pl = lin / ((int64_t)ti_n * tj_n);
    const int trem = (int)(lin % ((int64_t)ti_n * tj_n));
    const int i0 = (trem / tj_n) * TI;
    const int j0 = (trem % tj_n) * TJ;
    Ab = pa + pl * plane_ax + (LT ? (int64_t)i0 : (int64_t)i0 * Np);
    Bb = pb + pl * plane + (RT ? (int64_t)j0 : (int64_t)j0 * Np);
    X = px + pl * plane_ax + (int64_t)i0 * Np + j0;
  };
  auto issue = [&](int stage, int k0) {
    const bf16* As = Ab + (LT ? (int64_t)k0 * Np : (int64_t)k0);
    const bf16* Bs = Bb + (RT ? (int64_t)k0 * Np : (int64_t)k0);
#pragma unroll
    for (int u = 0; u < RA; ++u)
      g2lds16_sv(As, voA[u], lds_a + (uint32_t)((stage * TI * BK + (wave + u * NW) * 512) * 2));
#pragma unroll
    for (int u = 0; u < RB; ++u)
      g2lds16_sv(Bs, voB[u], lds_b + (uint32_t)((stage * TJ * BK + (wave + u * NW) * 512) * 2));
  };
  // fragment of a transposed panel (cols columns a row): lane l takes column
  // c0 + (l & 31), k 16 kc + 8 (l >> 5) .. +7
  auto tfrag = [&](const bf16* panel, int cols, int c0, int kc) {
    const int G = lane >> 4, sl = lane & 15;
    const int col = c0 + 16 * (G & 1) + 4 * (sl & 3);  // this lane's supplier column (4 elements)
    const int k0 = 16 * kc + 8 * (G >> 1) + (sl >> 2);  // and row, first read
    auto at = [&](int r) { return panel + r * cols + 8 * ((col >> 3) ^ tswz(r)) + (col & 7); };
    typedef short s16x8 __attribute__((ext_vector_type(8)));
    const s16x4 p0 = lds_read_tr16(at(k0)), p1 = lds_read_tr16(at(k0 + 4));
    Frag<bf16> f;
    f.v = __builtin_bit_cast(bf16x8, s16x8{p0[0], p0[1], p0[2], p0[3], p1[0], p1[1], p1[2], p1[3]});
    return f;
  };
  constexpr int kStores = 8;  // store instructions per wave and tile

  const int KT = Np / BK;  // Np is a multiple of 128: KT >= 2 and even
  int64_t v = blockIdx.x;
  if (v >= total) return;  // block-uniform
  setup(v);
  issue(0, 0);
  bool first = true;
  for (; v < total; v += gridDim.x) {
    bf16* const Xt = X;
    f32x16 acc[2][2];
#pragma unroll
    for (int x = 0; x < 2; ++x)
#pragma unroll
      for (int y = 0; y < 2; ++y) acc[x][y] = zero16();
    for (int kt = 0; kt < KT; ++kt) {
      // this wave's copies of stage kt landed: behind the first stage's
      // copies are, after the first tile, the previous tile's stores
      if (kt == 0 && !first) __builtin_amdgcn_s_waitcnt(vmcnt_imm<kStores>());
      else __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
      barrier_only();  // stage kt visible to every wave; stage kt-1 fully consumed
      if (kt + 1 < KT) {
        issue((kt + 1) % NS, (kt + 1) * BK);
      } else if (v + gridDim.x < total) {
        setup(v + gridDim.x);  // stage 0 (KT even) was consumed at kt - 1
        issue(0, 0);
      }
      const bf16* sa = ring + (kt % NS) * TI * BK;
      const bf16* sb = ring + NS * TI * BK + (kt % NS) * TJ * BK;
      // fragments of all k chunks are read up front so later chunks' reads
      // overlap the earlier chunks' MFMAs
      Frag<bf16> fa[BK / 16][2], fb[BK / 16][2];
#pragma unroll
      for (int kc = 0; kc < BK / 16; ++kc) {
        const int lc = kc * 2 + half;
#pragma unroll
        for (int x = 0; x < 2; ++x) {
          const int r_a = wi + x * 32 + (lane & 31);
          const int r_b = wj + x * 32 + (lane & 31);
          if constexpr (LT) fa[kc][x] = tfrag(sa, TI, wi + x * 32, kc);
          else fa[kc][x].load(sa + r_a * BK + 8 * (lc ^ pswz(r_a)));
          if constexpr (RT) fb[kc][x] = tfrag(sb, TJ, wj + x * 32, kc);
          else fb[kc][x].load(sb + r_b * BK + 8 * (lc ^ pswz(r_b)));
        }
      }
#pragma unroll
      for (int kc = 0; kc < BK / 16; ++kc)
#pragma unroll
        for (int x = 0; x < 2; ++x)
#pragma unroll
          for (int y = 0; y < 2; ++y) mma(acc[x][y], fb[kc][y], fa[kc][x]);  // rows j, cols i
    }
    first = false;
    // acc[x][y]: lane (t, h) holds X[wi + 32x + t][wj + 32y + 8g + 4h + r].
    // The half-waves swap quads (v_permlane32_swap) so that the lower half
    // holds columns 16p .. 16p+7 and the upper half 16p+8 .. 16p+15 of pair p
    // of quads: one 16-byte store per lane writes 32 contiguous bytes of each
    // of 32 rows.
#pragma unroll
    for (int x = 0; x < 2; ++x)
#pragma unroll
      for (int y = 0; y < 2; ++y) {
        uint32_t lo[4], hi[4];  // columns 8g + 4h + {0,1} and {2,3}
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          lo[g] = pack_bf16x2(acc[x][y][4 * g], acc[x][y][4 * g + 1]);
          hi[g] = pack_bf16x2(acc[x][y][4 * g + 2], acc[x][y][4 * g + 3]);
        }
        bf16* row = Xt + (int64_t)(wi + 32 * x + (lane & 31)) * Np + wj + 32 * y;
#pragma unroll
        for (int p = 0; p < 2; ++p) {
          // lower lanes receive the upper half's quad 2p, upper lanes the
          // lower half's quad 2p + 1
          const auto sl = __builtin_amdgcn_permlane32_swap(lo[2 * p], lo[2 * p + 1], false, false);
          const auto sh = __builtin_amdgcn_permlane32_swap(hi[2 * p], hi[2 * p + 1], false, false);
          const uint4 val = half ? make_uint4(sl[0], sh[0], lo[2 * p + 1], hi[2 * p + 1])
                                 : make_uint4(lo[2 * p], hi[2 * p], sl[1], sh[1]);
          *reinterpret_cast<uint4*>(row + 16 * p + 8 * half) = val;
        }
      }
  }
}

// ---------------------------------------------------------------------------
// 2c. fp8 contraction (the fp8 a/b storage experiment): A and Bm planes in
//     OCP fp8 E4M3 (1 byte per element), X in bf16.  The bf16 kernel's
//     structure with stages of 128 k (128-byte panel rows, the same geometry
//     and swizzle) and v_mfma_f32_32x32x64_f8f6f4: each lane feeds 32 bytes
//     of its row per operand, and the A and B lanes of a half-wave read the
//     same k bytes, so every product pairs A and B at the same k whatever the
//     instruction's internal slot order.  Np % 256 == 0.
// ---------------------------------------------------------------------------
template <int TI, int TJ>
__global__ __launch_bounds__(64 * (TI / 64) * (TJ / 64)) void trimul_contract_fp8_kernel(
    const uint8_t* __restrict__ pa, const uint8_t* __restrict__ pb, bf16* __restrict__ px, int Np,
    int64_t nplanes, int64_t plane, int64_t plane_x) {
  constexpr int BK = 128, NS = 2;                   // k per stage = bytes per panel row
  constexpr int NW = (TI / 64) * (TJ / 64);         // waves
  constexpr int RPR = 1024 / BK;                    // panel rows per 1 KiB copy
  constexpr int CPR = BK / 16;                      // 16-byte chunks per panel row
  static_assert((TI / RPR) % NW == 0 && (TJ / RPR) % NW == 0, "copies split evenly");
  typedef int v8i __attribute__((ext_vector_type(8)));
  typedef int v4i __attribute__((ext_vector_type(4)));
  __shared__ __attribute__((aligned(1024))) uint8_t ring[NS * (TI + TJ) * BK];
  uint8_t(*ra_l)[TI * BK] = reinterpret_cast<uint8_t(*)[TI * BK]>(ring);
  uint8_t(*rb_l)[TJ * BK] = reinterpret_cast<uint8_t(*)[TJ * BK]>(ring + NS * TI * BK);

  const int ti_n = Np / TI, tj_n = Np / TJ;
  const int64_t total = (int64_t)ti_n * tj_n * nplanes;
  const int64_t lin = xcd_remap((int64_t)blockIdx.x, total);
  const int64_t pl = lin / ((int64_t)ti_n * tj_n);
  const int trem = (int)(lin % ((int64_t)ti_n * tj_n));
  const int i0 = (trem / tj_n) * TI;
  const int j0 = (trem % tj_n) * TJ;
  const uint8_t* A = pa + pl * plane;
  const uint8_t* Bm = pb + pl * plane;

  const int lane = threadIdx.x & 63;
  const int wave = wave_id();
  const int half = lane >> 5;
  const int wi = (wave / (TJ / 64)) * 64;
  const int wj = (wave % (TJ / 64)) * 64;
  auto pswz = [](int r) { return (r ^ (r >> 3)) & 7; };

  constexpr int RA = TI / RPR / NW, RB = TJ / RPR / NW;
  const uint8_t* srcA[RA];
  const uint8_t* srcB[RB];
#pragma unroll
  for (int u = 0; u < RA; ++u) {
    const int row = RPR * (wave + u * NW) + lane / CPR;
    srcA[u] = A + (int64_t)(i0 + row) * Np + 16 * ((lane % CPR) ^ pswz(row));
  }
#pragma unroll
  for (int u = 0; u < RB; ++u) {
    const int row = RPR * (wave + u * NW) + lane / CPR;
    srcB[u] = Bm + (int64_t)(j0 + row) * Np + 16 * ((lane % CPR) ^ pswz(row));
  }
  auto issue = [&](int stage, int k0) {
#pragma unroll
    for (int u = 0; u < RA; ++u) g2lds16(srcA[u] + k0, &ra_l[stage][(wave + u * NW) * 1024]);
#pragma unroll
    for (int u = 0; u < RB; ++u) g2lds16(srcB[u] + k0, &rb_l[stage][(wave + u * NW) * 1024]);
  };
  // 32 bytes of panel row r: logical chunks 2m, 2m+1 (m = 2 kc + half)
  auto frag = [&](const uint8_t* base, int r, int m) {
    const v4i lo = *reinterpret_cast<const v4i*>(base + r * BK + 16 * ((2 * m) ^ pswz(r)));
    const v4i hi = *reinterpret_cast<const v4i*>(base + r * BK + 16 * ((2 * m + 1) ^ pswz(r)));
    return v8i{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
  };

  f32x16 acc[2][2];
#pragma unroll
  for (int x = 0; x < 2; ++x)
#pragma unroll
    for (int y = 0; y < 2; ++y) acc[x][y] = zero16();

  const int KT = Np / BK;  // Np % 256 == 0: KT >= 2
  issue(0, 0);
  for (int kt = 0; kt < KT; ++kt) {
    __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): this wave's copies of stage kt landed
    barrier_only();  // stage kt visible to every wave; stage kt-1 fully consumed
    if (kt + 1 < KT) issue((kt + 1) % NS, (kt + 1) * BK);
    const uint8_t* sa = ra_l[kt % NS];
    const uint8_t* sb = rb_l[kt % NS];
    v8i fa[BK / 64][2], fb[BK / 64][2];
#pragma unroll
    for (int kc = 0; kc < BK / 64; ++kc)
#pragma unroll
      for (int x = 0; x < 2; ++x) {
        fa[kc][x] = frag(sa, wi + x * 32 + (lane & 31), 2 * kc + half);
        fb[kc][x] = frag(sb, wj + x * 32 + (lane & 31), 2 * kc + half);
      }
#pragma unroll
    for (int kc = 0; kc < BK / 64; ++kc)
#pragma unroll
      for (int x = 0; x < 2; ++x)
#pragma unroll
        for (int y = 0; y < 2; ++y)  // rows j, cols i; formats: fp8 E4M3 for both operands
          acc[x][y] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(fb[kc][y], fa[kc][x], acc[x][y],
                                                                      0, 0, 0, 0, 0, 0);
  }

  // the bf16 kernel's output path: transpose through the ring, whole rows out
  constexpr int CPO = TJ / 8;
  static_assert(TI * TJ * 2 <= NS * (TI + TJ) * BK, "output tile fits in the ring");
  static_assert(CPO >= 16 && (64 * NW) % CPO == 0 && TI % (64 * NW / CPO) == 0, "store split");
  bf16* tl = reinterpret_cast<bf16*>(ring);
  barrier_only();
#pragma unroll
  for (int x = 0; x < 2; ++x) {
    const int il = wi + x * 32 + (lane & 31);
#pragma unroll
    for (int y = 0; y < 2; ++y)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int jl = wj + y * 32 + 8 * g + 4 * half;
        store4(tl + il * TJ + ((((jl >> 3) ^ (il & (CPO - 1))) << 3) | (jl & 7)), acc[x][y][4 * g + 0],
               acc[x][y][4 * g + 1], acc[x][y][4 * g + 2], acc[x][y][4 * g + 3]);
      }
  }
  barrier_only();
  bf16* X = px + pl * plane_x;
  constexpr int RPI = 64 * NW / CPO;
  const int rr = (int)threadIdx.x / CPO, cc = (int)threadIdx.x % CPO;
#pragma unroll
  for (int r0 = 0; r0 < TI; r0 += RPI) {
    const int r = r0 + rr;
    const uint4 v = *reinterpret_cast<const uint4*>(tl + r * TJ + ((cc ^ (r & (CPO - 1))) << 3));
    *reinterpret_cast<uint4*>(X + (int64_t)(i0 + r) * Np + j0 + cc * 8) = v;
  }
}

// ---------------------------------------------------------------------------
// 3. Epilogue
//    Both epilogues produce output rows i = r0 .. r0 + nrows - 1 from rows
//    i - r0 of the x planes, which hold xrows x Np (whole planes: r0 = 0,
//    nrows = N, xrows = Np).
// ---------------------------------------------------------------------------
template <typename T, int CZ, int CH>
__global__ __launch_bounds__(256) void trimul_epilogue_kernel(
    const T* __restrict__ z, const T* __restrict__ px, T* __restrict__ out, TriMulPacked<T> w,
    int B, int N, int Np, int residual, float eps_in, float eps_out, int r0, int nrows, int xrows,
    int64_t plane) {
  constexpr int XPITCH = CH + 8;  // LDS row pitch (elements) of the transposed x tile
  __shared__ __attribute__((aligned(16))) T xs[4][32 * XPITCH];
  const int lane = threadIdx.x & 63;
  const int wave = wave_id();
  const int half = lane >> 5;
  const int t32 = lane & 31;
  const int jtiles = (N + 31) / 32;
  const int64_t tile = (int64_t)blockIdx.x * 4 + wave;
  if (tile >= (int64_t)B * nrows * jtiles) return;
  const int jt = (int)(tile % jtiles);
  const int il = (int)((tile / jtiles) % nrows);  // row of the x planes
  const int i = r0 + il;
  const int b = (int)(tile / ((int64_t)jtiles * nrows));
  const int j = jt * 32 + t32;
  const bool valid = j < N;
  const int64_t pair = ((int64_t)b * N + i) * N + (valid ? j : 0);

  // Gate from z.
  f32x16 gate[CZ / 32];
  {
    RowHalf<CZ> rh;
    load_row_half<T, CZ>(rh, z + pair * CZ, valid);
    const f32x2 st = row_stats<CZ>(rh, eps_in);
    Frag<T> xf[CZ / 16];
    if constexpr (trimul_folded<CZ, CH>()) ln_to_frags<T, CZ>(xf, rh, st);
    else ln_affine_to_frags<T, CZ>(xf, rh, st, w.ln_in_w, w.ln_in_b);
#pragma unroll
    for (int nt = 0; nt < CZ / 32; ++nt) {
      gate[nt] = row_gemm_tile<T, CZ, true>(xf, w.w_g, nt);
#pragma unroll
      for (int g = 0; g < 4; ++g)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int c = nt * 32 + 8 * g + 4 * half + r;
          gate[nt][4 * g + r] = gate_from_u(gate[nt][4 * g + r] + w.b_g[c]);
        }
    }
  }

  // Transpose the x tile X[b][c][i][jt*32 .. +32] through LDS into [j][c].
  {
    constexpr int EPC = 16 / sizeof(T);   // elements per 16-byte chunk
    constexpr int CPR = 32 / EPC;         // chunks per c-row of 32 elements
    constexpr int TOTAL = CH * CPR;
    const T* xb = px + (int64_t)b * CH * plane + (int64_t)il * Np + jt * 32;
    T* s = xs[wave];
#pragma unroll 4
    for (int id = lane; id < TOTAL; id += 64) {
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
    const T* s = xs[wave] + t32 * XPITCH + half * (CH / 2);
#pragma unroll
    for (int ch = 0; ch < CH / 16; ++ch) {
      Frag<T> f;
      f.load(s + ch * 8);
#pragma unroll
      for (int e = 0; e < 8; ++e) xh.v[ch * 8 + e] = f.get(e);
    }
  }
  const f32x2 st = row_stats<CH>(xh, eps_out);
  Frag<T> yf[CH / 16];
  if constexpr (trimul_folded<CZ, CH>()) ln_to_frags<T, CH>(yf, xh, st);
  else ln_affine_to_frags<T, CH>(yf, xh, st, w.ln_out_w, w.ln_out_b);

#pragma unroll
  for (int nt = 0; nt < CZ / 32; ++nt) {
    const f32x16 acc = row_gemm_tile<T, CH, true>(yf, w.w_z, nt);
    if (valid) {
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int c0 = nt * 32 + 8 * g + 4 * half;
        float o[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) o[r] = (acc[4 * g + r] + w.b_z[c0 + r]) * gate[nt][4 * g + r];
        if (residual) {
          const f32x4 zr = load4f(z + pair * CZ + c0);
#pragma unroll
          for (int r = 0; r < 4; ++r) o[r] += zr[r];
        }
        store4(out + pair * CZ + c0, o[0], o[1], o[2], o[3]);
      }
    }
  }
}

// ---------------------------------------------------------------------------
// 3b. bf16 epilogue: persistent, 8 waves per CU with W_g and W_z resident in
//     LDS.  Per 32-pair tile (row i, pairs jt*32 ..):
//   * the x tile (c rows of 32 pairs, 64 B each) lands in the wave's own LDS
//     buffer with direct global->LDS copies, chunk-swizzled so the transposing
//     reads below are bank-conflict free, and is read back with
//     ds_read_b64_tr_b16 straight into MFMA fragments (lane = pair, 8
//     consecutive channels per fragment);
//   * the next tile's x copy and z row loads are issued before this tile's
//     matrix work, so their latency hides behind it;
//   * gate = sigmoid(LN_in(z) W_g^T + b_g) and (LN_out(x) W_z^T + b_z) are
//     produced one 32-channel tile at a time and multiplied;
//   * each 32-channel tile of the result goes through the wave's 2 KiB LDS
//     region ([pair][32 channels], 16-byte chunk k of pair p at physical chunk
//     k ^ (p & 3)) and leaves as two 16-byte-per-lane stores, each 16 pairs x
//     64 contiguous bytes, instead of four 8-byte stores per lane that touch a
//     cache line per pair (52.8 -> 51.6 us at N = 512, bit-identical output).
//   * RES (the residual add) is a template parameter: as a run-time flag the
//     compiler computed both sums of every output and selected one.
// ---------------------------------------------------------------------------
template <int CZ, int CH, bool RES>
__global__ __launch_bounds__(512) void trimul_epilogue_bf16_kernel(
    const bf16* __restrict__ z, const bf16* __restrict__ px, bf16* __restrict__ out,
    TriMulPacked<bf16> w, int N, int Np, float eps_in, float eps_out,
    int64_t ntiles, int r0, int nrows, int xrows, int64_t plane) {
  constexpr bool residual = RES;
  constexpr int WAVES = 8;
  constexpr int KZ = CZ / 16;                 // k chunks over c_z (gate input)
  constexpr int KX = CH / 16;                 // k chunks over c (W_z input)
  constexpr int PG = (CZ / 32) * KZ * 512;    // packed W_g elements
  constexpr int PZ = (CZ / 32) * KX * 512;    // packed W_z elements
  __shared__ __attribute__((aligned(1024))) bf16 wl[PG + PZ];
  __shared__ __attribute__((aligned(1024))) bf16 xt[WAVES][CH * 32];
  __shared__ __attribute__((aligned(16))) float bl[2 * CZ];
  __shared__ __attribute__((aligned(1024))) char stg[WAVES][2048];  // one output tile per wave
  copy_to_lds_async(wl, w.w_g, PG * 2);
  copy_to_lds_async(wl + PG, w.w_z, PZ * 2);
  for (int t = threadIdx.x; t < CZ; t += blockDim.x) {
    bl[t] = w.b_g[t];
    bl[CZ + t] = w.b_z[t];
  }
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();

  const int lane = threadIdx.x & 63;
  const int wave = wave_id();
  const int half = lane >> 5;
  const int t32 = lane & 31;
  const int jtiles = (N + 31) / 32;
  bf16* xw = xt[wave];
  const bf16* wg = wl;
  const bf16* wz = wl + PG;
  char* const sw = stg[wave];

  // x tile in LDS: channel row c at xw + 32c, physical 16-byte chunk p holds
  // pairs 8k .. 8k+7 with k = p ^ swz(c).  Copy instruction n moves rows
  // 16n .. 16n+15; lane l lands at row 16n + l/4, physical chunk l%4.
  auto swz = [](int c) { return 2 * ((c >> 1) & 1); };
  // tiles: [B][nrows rows i - r0][jtiles], walked without divisions
  auto issue_x = [&](const TileWalk& tw) {
    const int jt = tw.c, il = tw.r, b = tw.b;
    const bf16* src = px + (int64_t)b * CH * plane + (int64_t)il * Np + jt * 32;
#pragma unroll
    for (int n = 0; n < CH / 16; ++n) {
      const int row = 16 * n + (lane >> 2);
      const int k = (lane & 3) ^ swz(row);
      g2lds16(src + row * plane + 8 * k, xw + n * 512);
    }
  };
  // Always KZ load instructions (an invalid pair reads pair j = 0; its
  // results are never stored): the wait below counts them.
  auto load_z = [&](Frag<bf16>* zr, const TileWalk& tw) {
    const int jt = tw.c, i = r0 + tw.r, b = tw.b;
    const int j = jt * 32 + t32;
    const bool valid = j < N;
    const bf16* row = z + (((int64_t)b * N + i) * N + (valid ? j : 0)) * CZ + half * (CZ / 2);
#pragma unroll
    for (int ch = 0; ch < KZ; ++ch) zr[ch].load(row + ch * 8);
  };
  // transposing-read addresses: fetching lane (group G = lane/16, i = lane%16)
  // reads channel row c_m, m = i/4, at pairs 16*(G&1) + 4*(i%4) .. +3
  const int G = lane >> 4;
  const int fm = (lane & 15) >> 2;
  const int fq = lane & 3;
  const int fk = 2 * (G & 1) + (fq >> 1);      // logical chunk
  const int fsub = 4 * (fq & 1);               // element offset inside the chunk
  auto read_x = [&](Frag<bf16>* xr) {
#pragma unroll
    for (int ks = 0; ks < KX; ++ks) {
      s16x4 part[2];
#pragma unroll
      for (int hh = 0; hh < 2; ++hh) {
        const int c = (G >> 1) * (CH / 2) + ks * 8 + hh * 4 + fm;
        part[hh] = lds_read_tr16(xw + c * 32 + 8 * (fk ^ swz(c)) + fsub);
      }
      const s16x4 lo = part[0], hi = part[1];
      typedef short s16x8 __attribute__((ext_vector_type(8)));
      const s16x8 v = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
      xr[ks].v = __builtin_bit_cast(bf16x8, v);
    }
  };

  int64_t tile = (int64_t)blockIdx.x * WAVES + wave;
  const int64_t stride = (int64_t)gridDim.x * WAVES;
  Frag<bf16> zr[KZ];
  // One tile.  The first tile is peeled off the loop (first = true) so that
  // every path into the loop has the previous tile's stores outstanding
  // behind the prefetched loads, and the waits can count them exactly.
  auto body = [&](const int64_t tile, const TileWalk& tw, const bool first) {
    const int jt = tw.c, i = r0 + tw.r, b = tw.b;
    const int nin = N - jt * 32;  // pairs of this tile inside the grid
    // this tile's 32 output pairs, one buffer range: every lane stores
    // (invalid pairs are dropped by the range check), no branch
    const auto orsrc = buf_rsrc(out + (((int64_t)b * N + i) * N + jt * 32) * CZ, 32 * CZ * 2);
    Frag<bf16> xf[KZ], yf[KX];
    ln_frags_bf16<CZ>(xf, zr, eps_in);
    // Residual z in the accumulator layout, taken from the rows just loaded:
    // output group q (channels 8q + 4*half + 0..3) sits in dwords 0-1
    // (q < KZ) or 2-3 (q >= KZ) of zr[q mod KZ] once dwords 2-3 of the lower
    // half-wave are swapped with dwords 0-1 of the upper one.
    bf16x4 zres[2 * KZ];
    if constexpr (residual) {
#pragma unroll
      for (int ch = 0; ch < KZ; ++ch) {
        typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
        typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
        const u32x4 d = __builtin_bit_cast(u32x4, zr[ch].v);
        const auto s02 = __builtin_amdgcn_permlane32_swap(d[0], d[2], false, false);
        const auto s13 = __builtin_amdgcn_permlane32_swap(d[1], d[3], false, false);
        zres[ch] = __builtin_bit_cast(bf16x4, u32x2{s02[0], s13[0]});
        zres[ch + KZ] = __builtin_bit_cast(bf16x4, u32x2{s02[1], s13[1]});
      }
    }
    // This tile's x copy has landed once at most the ops issued after it are
    // outstanding: the KZ row loads, then (after the first tile) the previous
    // tile's 2*CZ/32 stores.  Loads complete in issue order, so the stores
    // need not have completed.
    if (first) __builtin_amdgcn_s_waitcnt(vmcnt_imm<KZ>());
    else __builtin_amdgcn_s_waitcnt(vmcnt_imm<KZ + 2 * (CZ / 32)>());
    {
      Frag<bf16> xr[KX];
      read_x(xr);
      ln_frags_bf16<CH>(yf, xr, eps_out);
    }
    __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): transposing reads done, the buffer is free
    if (tile + stride < ntiles) {
      TileWalk nx = tw;
      nx.next();
      issue_x(nx);
      load_z(zr, nx);
    }
    // unrolled: zres is indexed by nt (a run-time index would put it in scratch)
#pragma unroll
    for (int nt = 0; nt < CZ / 32; ++nt) {
      Frag<bf16> f;
      load_wfrag_lds(f, wg, nt, 0, KZ);
      f32x16 ga = mma0(f, xf[0]);
#pragma unroll
      for (int ks = 1; ks < KZ; ++ks) {
        load_wfrag_lds(f, wg, nt, ks, KZ);
        mma(ga, f, xf[ks]);
      }
      load_wfrag_lds(f, wz, nt, 0, KX);
      f32x16 oa = mma0(f, yf[0]);
#pragma unroll
      for (int ks = 1; ks < KX; ++ks) {
        load_wfrag_lds(f, wz, nt, ks, KX);
        mma(oa, f, yf[ks]);
      }
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int c0 = nt * 32 + 8 * g + 4 * half;
        const f32x4 bg = *reinterpret_cast<const f32x4*>(bl + c0);
        const f32x4 bz = *reinterpret_cast<const f32x4*>(bl + CZ + c0);
        float o[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          o[r] = (oa[4 * g + r] + bz[r]) * gate_from_u(ga[4 * g + r] + bg[r]);
          if constexpr (residual) o[r] += (float)zres[nt * 4 + g][r];
        }
        typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
        *reinterpret_cast<u32x2*>(sw + t32 * 64 + ((g ^ (t32 & 3)) << 4) + half * 8) =
            u32x2{pack_bf16x2(o[0], o[1]), pack_bf16x2(o[2], o[3])};
      }
      // lane l stores pair 16 k2 + l/4, channels nt*32 + 8 (l%4) .. +7
#pragma unroll
      for (int k2 = 0; k2 < 2; ++k2) {
        const int p = 16 * k2 + (lane >> 2), c = lane & 3;
        const uint4 v = *reinterpret_cast<const uint4*>(sw + p * 64 + ((c ^ (p & 3)) << 4));
        buf_store16(orsrc, p < nin ? (uint32_t)((p * CZ + nt * 32 + c * 8) * 2) : kBufSkip, v);
      }
      __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): read back before the next tile overwrites it
    }
  };
  TileWalk tw;
  tw.init(tile, stride, nrows, jtiles);
  if (tile < ntiles) {
    issue_x(tw);
    load_z(zr, tw);
    body(tile, tw, true);
    tile += stride;
    tw.next();
  }
  for (; tile < ntiles; tile += stride, tw.next()) body(tile, tw, false);
}

// ---------------------------------------------------------------------------
// Layout conversion for the raw contraction op:
//   pairs [B][N][N][C]  <->  planes [B][C][Np][Np]
// ---------------------------------------------------------------------------
template <typename T>
__global__ __launch_bounds__(256) void pairs_to_planes_kernel(const T* __restrict__ src,
                                                              T* __restrict__ dst, int B, int N,
                                                              int Np, int C, int outgoing) {
  const int lane = threadIdx.x & 63;
  const int half = lane >> 5;
  const int vtiles = Np / 32;
  const int64_t tile = (int64_t)blockIdx.x * 4 + wave_id();
  if (tile >= (int64_t)B * Np * vtiles) return;
  const int vt = (int)(tile % vtiles);
  const int f = (int)((tile / vtiles) % Np);
  const int b = (int)(tile / ((int64_t)vtiles * Np));
  const int v = vt * 32 + (lane & 31);
  const int p = outgoing ? f : v, q = outgoing ? v : f;
  const bool valid = p < N && q < N;
  const T* s = src + (((int64_t)b * N + (valid ? p : 0)) * N + (valid ? q : 0)) * C;
  const int64_t plane = (int64_t)Np * Np;
  T* d = dst + (int64_t)b * C * plane + (int64_t)f * Np + v;
  for (int c = half * (C / 2); c < (half + 1) * (C / 2); c += 8) {
    Frag<T> fr;
    if (valid) fr.load(s + c);
    else fr.zero();
#pragma unroll
    for (int e = 0; e < 8; ++e) d[(int64_t)(c + e) * plane] = cvt<T>(fr.get(e));
  }
}

template <typename T>
__global__ __launch_bounds__(256) void planes_to_pairs_kernel(const T* __restrict__ src,
                                                              T* __restrict__ dst, int B, int N,
                                                              int Np, int C) {
  const int lane = threadIdx.x & 63;
  const int half = lane >> 5;
  const int jtiles = (N + 31) / 32;
  const int64_t tile = (int64_t)blockIdx.x * 4 + wave_id();
  if (tile >= (int64_t)B * N * jtiles) return;
  const int jt = (int)(tile % jtiles);
  const int i = (int)((tile / jtiles) % N);
  const int b = (int)(tile / ((int64_t)jtiles * N));
  const int j = jt * 32 + (lane & 31);
  if (j >= N) return;
  const int64_t plane = (int64_t)Np * Np;
  const T* s = src + (int64_t)b * C * plane + (int64_t)i * Np + j;
  T* d = dst + (((int64_t)b * N + i) * N + j) * C;
  for (int c = half * (C / 2); c < (half + 1) * (C / 2); c += 8) {
    float f8[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) f8[e] = to_f32(s[(int64_t)(c + e) * plane]);
    Frag<T> fr;
    fr.set(f8);
    if constexpr (sizeof(T) == 2) {
      *reinterpret_cast<bf16x8*>(d + c) = fr.v;
    } else {
      *reinterpret_cast<f32x4*>(d + c) = fr.lo;
      *reinterpret_cast<f32x4*>(d + c + 4) = fr.hi;
    }
  }
}

// Output tile of the contraction for Np (a multiple of 64): row chunks are
// multiples of it.
// 256-row tiles need bf16 and Np % 256 == 0; with fewer than two of them per
// CU across the planes (small N), 128-row tiles keep every CU busy.
template <typename T>
static int contract_tile(int Np, int64_t nplanes = 1 << 20) {
  if (sizeof(T) == 2 && Np % 256 == 0 && (int64_t)(Np / 256) * (Np / 256) * nplanes >= 2 * device_cus())
    return 256;
  return Np % 128 == 0 ? 128 : 64;
}

// X = A . Bm^T per plane: A and X are Mi x Np (Mi a multiple of
// contract_tile(Np); Mi = Np for whole planes), Bm is Np x Np; plane strides
// ps_b (Bm) and ps_ax (A, X), by default the unpadded Np * Np and Mi * Np.
template <typename T>
static int launch_contract(const T* pa, const T* pb, T* px, int Np, int64_t nplanes,
                           hipStream_t st, int Mi = 0, int64_t ps_b = 0, int64_t ps_ax = 0) {
  if (Mi == 0) Mi = Np;
  if (ps_b == 0) ps_b = (int64_t)Np * Np;
  if (ps_ax == 0) ps_ax = (int64_t)Mi * Np;
  const int tile = contract_tile<T>(Np, nplanes);
  GTK_REQUIRE(Mi > 0 && Mi % tile == 0 && Mi <= Np, GTK_EINVAL, "contraction: %d rows, tile %d", Mi, tile);
  const int64_t blocks = (int64_t)(Mi / tile) * (Np / tile) * nplanes;
  GTK_REQUIRE(blocks < (1ll << 31), GTK_EUNSUPPORTED, "contraction grid too large");
  StageTimer timer("trimul_contract", st);
  // the bf16 kernel is persistent: one 256x256 block or two 128x128 blocks
  // per CU (LDS), a multiple of 8 blocks unless there are fewer tiles
  if (tile == 256) {
    const int64_t grid = std::min<int64_t>(blocks, device_cus());
    trimul_contract_bf16_kernel<256, 256><<<(unsigned)grid, 1024, 0, st>>>(
        (const bf16*)pa, (const bf16*)pb, (bf16*)px, Np, Mi, nplanes, ps_b, ps_ax);
  } else if (tile == 128) {
    const int64_t grid = std::min<int64_t>(blocks, 2 * device_cus());
    if constexpr (sizeof(T) == 2)
      trimul_contract_bf16_kernel<128, 128><<<(unsigned)grid, 256, 0, st>>>(pa, pb, px, Np, Mi, nplanes,
                                                                             ps_b, ps_ax);
    else
      trimul_contract_kernel<T, 128><<<(unsigned)blocks, 256, 0, st>>>(pa, pb, px, Np, Mi, nplanes, ps_b, ps_ax);
  } else {
    trimul_contract_kernel<T, 64><<<(unsigned)blocks, 256, 0, st>>>(pa, pb, px, Np, Mi, nplanes, ps_b, ps_ax);
  }
  GTK_LAUNCH_CHECK();
  return GTK_OK;
}

static size_t plane_bytes(int64_t B, int64_t N, int64_t C, int dtype) {
  const int64_t Np = round_up(N, 64);
  return (size_t)(B * C * Np * Np) * dtype_size(dtype);
}

template <typename T>
static int raw_contract(const void* a, const void* b, void* x, int64_t B, int64_t N, int64_t C,
                        int outgoing, void* ws, hipStream_t st) {
  const int Np = (int)round_up(N, 64);
  Carve cv(ws, SIZE_MAX);
  T* pa = cv.take<T>(B * C * (int64_t)Np * Np);
  T* pb = cv.take<T>(B * C * (int64_t)Np * Np);
  T* px = cv.take<T>(B * C * (int64_t)Np * Np);
  const int64_t ptiles = B * (int64_t)Np * (Np / 32);
  const unsigned pgrid = (unsigned)((ptiles + 3) / 4);
  pairs_to_planes_kernel<T><<<pgrid, 256, 0, st>>>((const T*)a, pa, (int)B, (int)N, Np, (int)C, outgoing);
  GTK_LAUNCH_CHECK();
  pairs_to_planes_kernel<T><<<pgrid, 256, 0, st>>>((const T*)b, pb, (int)B, (int)N, Np, (int)C, outgoing);
  GTK_LAUNCH_CHECK();
  int rc = launch_contract<T>(pa, pb, px, Np, B * C, st);
  if (rc) return rc;
  const int64_t otiles = B * N * ((N + 31) / 32);
  planes_to_pairs_kernel<T><<<(unsigned)((otiles + 3) / 4), 256, 0, st>>>(px, (T*)x, (int)B, (int)N, Np, (int)C);
  GTK_LAUNCH_CHECK();
  return GTK_OK;
}

static int raw_trimul(const void* a, const void* b, const float* mask, void* x, int64_t B,
                      int64_t N, int64_t C, int dtype, void* ws, size_t ws_bytes, void* stream,
                      int outgoing) {
  (void)mask;
  const char* name = outgoing ? "gtk_triangle_mul_outgoing" : "gtk_triangle_mul_incoming";
  GTK_REQUIRE(dtype == GTK_F32 || dtype == GTK_BF16, GTK_EINVAL, "%s: bad dtype %d", name, dtype);
  GTK_REQUIRE(B >= 0 && N >= 0 && C >= 1, GTK_EINVAL, "%s: bad shape", name);
  GTK_REQUIRE(C % 16 == 0, GTK_EUNSUPPORTED, "%s: C=%lld must be a multiple of 16", name, (long long)C);
  GTK_REQUIRE(N <= 16384, GTK_EUNSUPPORTED, "%s: N=%lld too large", name, (long long)N);
  if (B == 0 || N == 0) return GTK_OK;
  GTK_REQUIRE(a && b && x && ws, GTK_EINVAL, "%s: null pointer", name);
  const size_t need = gtk_triangle_mul_workspace_size(B, N, C, dtype);
  GTK_REQUIRE(ws_bytes >= need, GTK_EWORKSPACE, "%s: workspace %zu < %zu bytes", name, ws_bytes, need);
  hipStream_t st = (hipStream_t)stream;
  if (dtype == GTK_F32) return raw_contract<float>(a, b, x, B, N, C, outgoing, ws, st);
  return raw_contract<bf16>(a, b, x, B, N, C, outgoing, ws, st);
}

// ---------------------------------------------------------------------------
// Fused forward
// ---------------------------------------------------------------------------
template <typename T>
static int pack_trimul(const gtk_tri_mul_weights* w, int cz, int c, void* packed, hipStream_t st) {
  PackScope batch(st);  // 16 packing launches issued as 3
  Carve cv(packed, SIZE_MAX);
  TriMulPacked<T> p = carve_trimul<T>(cv, cz, c);
  const int wd = w->dtype;
  int rc = 0;
  // fp32 LayerNorm parameters first: they are folded into what follows
  if ((rc = launch_to_f32(p.ln_in_w, w->ln_in_w, wd, cz, 1.f, 1.f, st))) return rc;
  if ((rc = launch_to_f32(p.ln_in_b, w->ln_in_b, wd, cz, 1.f, 0.f, st))) return rc;
  if ((rc = launch_to_f32(p.ln_out_w, w->ln_out_w, wd, c, 1.f, 1.f, st))) return rc;
  if ((rc = launch_to_f32(p.ln_out_b, w->ln_out_b, wd, c, 1.f, 0.f, st))) return rc;
  // nn.Linear weight [out][in]: s_out = in, s_in = 1.
  // Gate projections (a_g, b_g, g) are packed pre-scaled by -log2(e): the
  // kernels evaluate sigmoid(x) as 1 / (1 + 2^u) with u = -log2(e) x.
  struct Lin { T* dst; float* bdst; const void* wsrc; const void* bsrc; int out, in; const float *g, *beta; float scale; };
  const float gs = -kLog2e;
  // LayerNorm affine folded in, or left to the kernels (trimul_folded)
  const bool fold = trimul_folded_rt(cz, c);
  const float* gi = fold ? p.ln_in_w : nullptr;
  const float* bi = fold ? p.ln_in_b : nullptr;
  const float* go = fold ? p.ln_out_w : nullptr;
  const float* bo = fold ? p.ln_out_b : nullptr;
  const Lin lins[6] = {
      {p.w_ap, p.b_ap, w->a_p_w, w->a_p_b, c, cz, gi, bi, 1.f},
      {p.w_ag, p.b_ag, w->a_g_w, w->a_g_b, c, cz, gi, bi, gs},
      {p.w_bp, p.b_bp, w->b_p_w, w->b_p_b, c, cz, gi, bi, 1.f},
      {p.w_bg, p.b_bg, w->b_g_w, w->b_g_b, c, cz, gi, bi, gs},
      {p.w_g, p.b_g, w->g_w, w->g_b, cz, cz, gi, bi, gs},
      {p.w_z, p.b_z, w->z_w, w->z_b, cz, c, go, bo, 1.f}};
  for (const Lin& l : lins) {
    if ((rc = launch_pack<T>(l.dst, l.wsrc, wd, l.out, l.in, l.in, 1, l.scale, st, l.g))) return rc;
    if ((rc = launch_fold_bias(l.bdst, l.wsrc, l.bsrc, wd, l.beta, l.out, l.in, l.in, 1, l.scale, st)))
      return rc;
  }
  return batch.flush();
}

// The bf16 kernels with LDS-resident weights are built for the module's
// shapes c_z = 128, c in {64, 128}; every other supported shape (c_z in {32,
// 64, 128}, c in {32, 64, 128, 256}) and fp32 run the generic kernels.
template <typename T, int CZ, int CH>
constexpr bool trimul_fast() {
  return sizeof(T) == 2 && CZ == 128 && (CH == 64 || CH == 128);
}

// Prologue over plane rows r0 .. r0 + nrows - 1 (default: all Np rows) for
// sides side_lo .. side_hi - 1 (0: A, 1: Bm), into planes of stride ps
// (default: the unpadded nrows * Np).
template <typename T, int CZ, int CH>
static int launch_trimul_prologue(const void* z, const float* mask, const TriMulPacked<T>& w, T* pa,
                                  T* pb, int64_t B, int64_t N, int Np, int outgoing, float eps_in,
                                  hipStream_t st, int r0 = 0, int nrows = 0, int side_lo = 0,
                                  int side_hi = 2, int64_t ps = 0) {
  if (nrows == 0) nrows = Np;
  if (ps == 0) ps = (int64_t)nrows * Np;
  const int64_t ptiles = B * (int64_t)nrows * (Np / 32);
  if constexpr (trimul_fast<T, CZ, CH>()) {
    // two tiles a step (each weight fragment read from LDS feeds both tiles'
    // products) while that still gives every wave of the grid a step; one
    // tile a step below that (N = 256: 1024 two-tile steps for 2048 waves)
    const bool one = ptiles / 2 < (int64_t)device_cus() * 8;
    const int grid = (int)std::min<int64_t>(device_cus(), (ptiles / (one ? 1 : 2) + 3) / 4);
    StageTimer timer("trimul_prologue", st);
    const bool whole = r0 == 0 && nrows == Np && side_lo == 0 && side_hi == 2;
    auto go = [&](auto kern) {
      kern<<<grid, 512, 0, st>>>((const bf16*)z, mask, (bf16*)pa, (bf16*)pb, w, (int)N, Np, outgoing,
                                 eps_in, ptiles, r0, nrows, side_lo, side_hi, ps);
    };
    if (whole) {
      if (one) go(trimul_prologue_bf16_kernel<CZ, CH, false, false, 1>);
      else go(trimul_prologue_bf16_kernel<CZ, CH, false, false, 2>);
    } else {
      if (one) go(trimul_prologue_bf16_kernel<CZ, CH, false, true, 1>);
      else go(trimul_prologue_bf16_kernel<CZ, CH, false, true, 2>);
    }
  } else {
    StageTimer timer("trimul_prologue", st);
    trimul_prologue_kernel<T, CZ, CH><<<(unsigned)((ptiles + 3) / 4), 256, 0, st>>>(
        (const T*)z, mask, pa, pb, w, (int)B, (int)N, Np, outgoing, eps_in, r0, nrows, side_lo,
        side_hi, ps);
  }
  GTK_LAUNCH_CHECK();
  return GTK_OK;
}

// Epilogue for output rows r0 .. r0 + nrows - 1 from x planes of xrows x Np
// and stride ps_x (default: all N rows from whole, unpadded planes).
template <typename T, int CZ, int CH>
static int launch_trimul_epilogue(const void* z, const T* px, void* out, const TriMulPacked<T>& w,
                                  int64_t B, int64_t N, int Np, int residual, float eps_in,
                                  float eps_out, hipStream_t st, int r0 = 0, int nrows = 0,
                                  int xrows = 0, int64_t ps_x = 0) {
  if (nrows == 0) nrows = (int)N;
  if (xrows == 0) xrows = Np;
  if (ps_x == 0) ps_x = (int64_t)xrows * Np;
  const int64_t etiles = B * nrows * ((N + 31) / 32);
  if constexpr (trimul_fast<T, CZ, CH>()) {
    const int grid = (int)std::min<int64_t>(device_cus(), (etiles + 7) / 8);
    StageTimer timer("trimul_epilogue", st);
    auto kern = residual ? trimul_epilogue_bf16_kernel<CZ, CH, true> : trimul_epilogue_bf16_kernel<CZ, CH, false>;
    kern<<<grid, 512, 0, st>>>((const bf16*)z, (const bf16*)px, (bf16*)out, w, (int)N, Np, eps_in, eps_out,
                               etiles, r0, nrows, xrows, ps_x);
  } else {
    StageTimer timer("trimul_epilogue", st);
    trimul_epilogue_kernel<T, CZ, CH><<<(unsigned)((etiles + 3) / 4), 256, 0, st>>>(
        (const T*)z, px, (T*)out, w, (int)B, (int)N, Np, residual, eps_in, eps_out, r0, nrows,
        xrows, ps_x);
  }
  GTK_LAUNCH_CHECK();
  return GTK_OK;
}

// Rows per chunk of the memory-bounded mode: chunk_rows rounded up to the
// largest contraction tile for Np (a multiple of whichever tile a launch
// picks); Np (whole planes) when chunk_rows is 0 or covers Np.
template <typename T>
static int trimul_chunk_rows(int64_t N, int64_t chunk_rows) {
  const int Np = (int)round_up(N, 64);
  if (chunk_rows <= 0 || chunk_rows >= Np) return Np;
  return (int)std::min<int64_t>(round_up(chunk_rows, contract_tile<T>(Np)), Np);
}

// Forward.  Whole planes: A, Bm and X of B*c planes of Np x Np.  Row chunks
// (R < Np rows): Bm over all rows once, then per chunk of R output rows the
// chunk's A rows, an R x Np contraction and the epilogue of those rows; the
// workspace holds Bm and two R x Np plane sets.  Every element takes the same
// arithmetic either way, so chunked and whole outputs are bit-identical.
template <typename T, int CZ, int CH>
static int fwd_trimul(const void* z, const float* mask, void* out, const void* packed, int64_t B,
                      int64_t N, int outgoing, int residual, float eps_in, float eps_out, void* ws,
                      hipStream_t st, int64_t chunk_rows) {
  Carve pc((void*)packed, SIZE_MAX);
  TriMulPacked<T> w = carve_trimul<T>(pc, CZ, CH);
  const int Np = (int)round_up(N, 64);
  const int R = trimul_chunk_rows<T>(N, chunk_rows);
  // padded plane strides (plane_stride): Bm of Np rows, A and X of R rows
  const int64_t ps_b = plane_stride<T>(Np, Np), ps_a = plane_stride<T>(R, Np);
  Carve cv(ws, SIZE_MAX);
  T* pb = cv.take<T>(B * CH * ps_b);
  T* pa = cv.take<T>(B * CH * ps_a);
  T* px = cv.take<T>(B * CH * ps_a);
  int rc;
  if (R == Np) {
    if ((rc = launch_trimul_prologue<T, CZ, CH>(z, mask, w, pa, pb, B, N, Np, outgoing, eps_in, st, 0,
                                                Np, 0, 2, ps_b)))
      return rc;
    if ((rc = launch_contract<T>(pa, pb, px, Np, B * CH, st, Np, ps_b, ps_a))) return rc;
    return launch_trimul_epilogue<T, CZ, CH>(z, px, out, w, B, N, Np, residual, eps_in, eps_out, st,
                                             0, (int)N, Np, ps_a);
  }
  if ((rc = launch_trimul_prologue<T, CZ, CH>(z, mask, w, pa, pb, B, N, Np, outgoing, eps_in, st, 0,
                                              Np, 1, 2, ps_b)))
    return rc;
  for (int r0 = 0; r0 < N; r0 += R) {
    const int rows = std::min(R, Np - r0);  // a multiple of the contraction tile
    if ((rc = launch_trimul_prologue<T, CZ, CH>(z, mask, w, pa, pb, B, N, Np, outgoing, eps_in, st,
                                                r0, rows, 0, 1, ps_a)))
      return rc;
    if ((rc = launch_contract<T>(pa, pb, px, Np, B * CH, st, rows, ps_b, ps_a))) return rc;
    if ((rc = launch_trimul_epilogue<T, CZ, CH>(z, px, out, w, B, N, Np, residual, eps_in, eps_out,
                                                st, r0, std::min<int>(rows, (int)N - r0), rows, ps_a)))
      return rc;
  }
  return GTK_OK;
}

// fp8 a/b experiment: planes padded to Np = N rounded up to 256 (the fp8
// contraction's tile); the prologue writes fp8 a and b, the contraction bf16
// x, and the bf16 epilogue finishes as in the bf16 forward.
static int64_t fp8_np(int64_t N) { return round_up(N, 256); }

static int launch_contract_fp8(const uint8_t* pa, const uint8_t* pb, bf16* px, int Np, int64_t nplanes,
                               hipStream_t st, int64_t ps_ab = 0, int64_t ps_x = 0) {
  if (ps_ab == 0) ps_ab = (int64_t)Np * Np;
  if (ps_x == 0) ps_x = (int64_t)Np * Np;
  GTK_REQUIRE(Np % 256 == 0, GTK_EINVAL, "fp8 contraction: Np=%d not a multiple of 256", Np);
  const int64_t blocks = (int64_t)(Np / 256) * (Np / 256) * nplanes;
  GTK_REQUIRE(blocks < (1ll << 31), GTK_EUNSUPPORTED, "contraction grid too large");
  StageTimer timer("trimul_contract_fp8", st);
  trimul_contract_fp8_kernel<256, 256><<<(unsigned)blocks, 1024, 0, st>>>(pa, pb, px, Np, nplanes, ps_ab, ps_x);
  GTK_LAUNCH_CHECK();
  return GTK_OK;
}

template <int CZ, int CH>
static int fwd_trimul_fp8(const void* z, const float* mask, void* out, const void* packed, int64_t B,
                          int64_t N, int outgoing, int residual, float eps_in, float eps_out, void* ws,
                          hipStream_t st) {
  Carve pc((void*)packed, SIZE_MAX);
  TriMulPacked<bf16> w = carve_trimul<bf16>(pc, CZ, CH);
  const int Np = (int)fp8_np(N);
  const int64_t ps_ab = plane_stride<uint8_t>(Np, Np), ps_x = plane_stride<bf16>(Np, Np);
  Carve cv(ws, SIZE_MAX);
  uint8_t* pa = cv.take<uint8_t>(B * CH * ps_ab);
  uint8_t* pb = cv.take<uint8_t>(B * CH * ps_ab);
  bf16* px = cv.take<bf16>(B * CH * ps_x);
  {
    const int64_t ptiles = B * (int64_t)Np * (Np / 32);
    const int grid = (int)std::min<int64_t>(device_cus(), (ptiles / 2 + 3) / 4);
    StageTimer timer("trimul_prologue_fp8", st);
    trimul_prologue_bf16_kernel<CZ, CH, true><<<grid, 512, 0, st>>>(
        (const bf16*)z, mask, pa, pb, w, (int)N, Np, outgoing, eps_in, ptiles, 0, Np, 0, 2, ps_ab);
    GTK_LAUNCH_CHECK();
  }
  int rc;
  if ((rc = launch_contract_fp8(pa, pb, px, Np, B * CH, st, ps_ab, ps_x))) return rc;
  return launch_trimul_epilogue<bf16, CZ, CH>(z, px, out, w, B, N, Np, residual, eps_in, eps_out, st,
                                              0, (int)N, Np, ps_x);
}

template <typename T, int CZ, int CH>
static int recompute_planes(const void* z, const float* mask, const void* packed, int64_t B,
                            int64_t N, int outgoing, float eps_in, void* pa, void* pb, void* px,
                            hipStream_t st) {
  Carve pc((void*)packed, SIZE_MAX);
  TriMulPacked<T> w = carve_trimul<T>(pc, CZ, CH);
  const int Np = (int)round_up(N, 64);
  int rc = launch_trimul_prologue<T, CZ, CH>(z, mask, w, (T*)pa, (T*)pb, B, N, Np, outgoing,
                                             eps_in, st);
  if (rc) return rc;
  return launch_contract<T>((const T*)pa, (const T*)pb, (T*)px, Np, B * CH, st);
}

int trimul_recompute_planes(const void* z, const float* mask, const void* packed, int64_t B,
                            int64_t N, int64_t c_z, int64_t c, int outgoing, float eps_in,
                            int dtype, void* pa, void* pb, void* px, hipStream_t st) {
#define GTK_RP(CZ_, C_)                                                                          \
  if (c_z == CZ_ && c == C_)                                                                    \
    return dtype == GTK_F32                                                                     \
               ? recompute_planes<float, CZ_, C_>(z, mask, packed, B, N, outgoing, eps_in, pa, pb, px, st) \
               : recompute_planes<bf16, CZ_, C_>(z, mask, packed, B, N, outgoing, eps_in, pa, pb, px, st);
  GTK_RP(128, 128) GTK_RP(128, 64) GTK_RP(128, 32)
  GTK_RP(64, 128) GTK_RP(64, 64) GTK_RP(64, 32)
  GTK_RP(32, 128) GTK_RP(32, 64) GTK_RP(32, 32)
#undef GTK_RP
  set_error("tri-mul plane recompute: c_z=%lld c=%lld unsupported", (long long)c_z, (long long)c);
  return GTK_EUNSUPPORTED;
}

int trimul_contract_planes(const void* pl, const void* pr, void* out, int Np, int64_t nplanes,
                           int dtype, hipStream_t st) {
  if (dtype == GTK_F32)
    return launch_contract<float>((const float*)pl, (const float*)pr, (float*)out, Np, nplanes, st);
  return launch_contract<bf16>((const bf16*)pl, (const bf16*)pr, (bf16*)out, Np, nplanes, st);
}

bool trimul_contract_t_ok(int Np, int64_t nplanes, int dtype) {
  return dtype != GTK_F32 && contract_tile<bf16>(Np, nplanes) >= 128;
}

int trimul_contract_planes_t(const void* pl, const void* pr, void* out, int Np, int64_t nplanes, bool lt,
                             bool rt, hipStream_t st) {
  GTK_REQUIRE(trimul_contract_t_ok(Np, nplanes, GTK_BF16), GTK_EUNSUPPORTED,
              "transposed-operand contraction: Np %d", Np);
  const int tile = contract_tile<bf16>(Np, nplanes);
  const int64_t blocks = (int64_t)(Np / tile) * (Np / tile) * nplanes;
  GTK_REQUIRE(blocks < (1ll << 31), GTK_EUNSUPPORTED, "contraction grid too large");
  const int64_t ps = (int64_t)Np * Np;
  const bf16* a = (const bf16*)pl;
  const bf16* b = (const bf16*)pr;
  bf16* x = (bf16*)out;
  StageTimer timer("trimul_contract", st);
  auto go = [&](auto kern, int threads, int64_t most) {
    kern<<<(unsigned)std::min<int64_t>(blocks, most), threads, 0, st>>>(a, b, x, Np, Np, nplanes, ps, ps);
  };
  if (tile == 256) {
    if (lt && rt) go(trimul_contract_bf16_kernel<256, 256, true, true>, 1024, device_cus());
    else if (lt) go(trimul_contract_bf16_kernel<256, 256, true, false>, 1024, device_cus());
    else if (rt) go(trimul_contract_bf16_kernel<256, 256, false, true>, 1024, device_cus());
    else go(trimul_contract_bf16_kernel<256, 256>, 1024, device_cus());
  } else {
    if (lt && rt) go(trimul_contract_bf16_kernel<128, 128, true, true>, 256, 2 * device_cus());
    else if (lt) go(trimul_contract_bf16_kernel<128, 128, true, false>, 256, 2 * device_cus());
    else if (rt) go(trimul_contract_bf16_kernel<128, 128, false, true>, 256, 2 * device_cus());
    else go(trimul_contract_bf16_kernel<128, 128>, 256, 2 * device_cus());
  }
  GTK_LAUNCH_CHECK();
  return GTK_OK;
}

}  // namespace gtk

using namespace gtk;

extern "C" size_t gtk_triangle_mul_workspace_size(int64_t B, int64_t N, int64_t C, int dtype) {
  if (B < 0 || N < 0 || C < 0) return 0;
  return 3 * (plane_bytes(B, N, C, dtype) + 256);
}

extern "C" int gtk_triangle_mul_outgoing(const void* a, const void* b, const float* mask, void* x,
                                         int64_t B, int64_t N, int64_t C, int dtype, void* ws,
                                         size_t ws_bytes, void* stream) {
  return raw_trimul(a, b, mask, x, B, N, C, dtype, ws, ws_bytes, stream, 1);
}

extern "C" int gtk_triangle_mul_incoming(const void* a, const void* b, const float* mask, void* x,
                                         int64_t B, int64_t N, int64_t C, int dtype, void* ws,
                                         size_t ws_bytes, void* stream) {
  return raw_trimul(a, b, mask, x, B, N, C, dtype, ws, ws_bytes, stream, 0);
}

static bool trimul_shape_ok(int64_t cz, int64_t c) {
  return (cz == 32 || cz == 64 || cz == 128) && (c == 32 || c == 64 || c == 128 || c == 256);
}

template <typename T>
static int fwd_trimul_any(int64_t cz, int64_t c, const void* z, const float* mask, void* out,
                          const void* packed, int64_t B, int64_t N, int outgoing, int residual,
                          float eps_in, float eps_out, void* ws, hipStream_t st, int64_t chunk_rows) {
#define GTK_TM(CZ_, C_)                                                                          \
  if (cz == CZ_ && c == C_)                                                                     \
    return fwd_trimul<T, CZ_, C_>(z, mask, out, packed, B, N, outgoing, residual, eps_in, eps_out, \
                                  ws, st, chunk_rows);
  GTK_TM(128, 128) GTK_TM(128, 64) GTK_TM(128, 32) GTK_TM(128, 256)
  GTK_TM(64, 128) GTK_TM(64, 64) GTK_TM(64, 32) GTK_TM(64, 256)
  GTK_TM(32, 128) GTK_TM(32, 64) GTK_TM(32, 32) GTK_TM(32, 256)
#undef GTK_TM
  set_error("tri-mul: c_z=%lld c=%lld unsupported", (long long)cz, (long long)c);
  return GTK_EUNSUPPORTED;
}

extern "C" size_t gtk_tri_mul_packed_size(int64_t c_z, int64_t c, int dtype) {
  if (!trimul_shape_ok(c_z, c)) return 0;
  Carve cv(nullptr, SIZE_MAX);
  if (dtype == GTK_F32) carve_trimul<float>(cv, (int)c_z, (int)c);
  else carve_trimul<bf16>(cv, (int)c_z, (int)c);
  return cv.off;
}

extern "C" int gtk_tri_mul_pack(const gtk_tri_mul_weights* w, int64_t c_z, int64_t c, int dtype,
                                void* packed, size_t packed_bytes, void* stream) {
  GTK_REQUIRE(w && packed, GTK_EINVAL, "gtk_tri_mul_pack: null pointer");
  GTK_REQUIRE(dtype == GTK_F32 || dtype == GTK_BF16, GTK_EINVAL, "gtk_tri_mul_pack: bad dtype %d", dtype);
  GTK_REQUIRE(w->dtype == GTK_F32 || w->dtype == GTK_BF16, GTK_EINVAL,
              "gtk_tri_mul_pack: bad weight dtype %d", w->dtype);
  GTK_REQUIRE(trimul_shape_ok(c_z, c), GTK_EUNSUPPORTED,
              "gtk_tri_mul_pack: c_z=%lld c=%lld unsupported (c_z in {32,64,128}, c in {32,64,128,256})",
              (long long)c_z, (long long)c);
  GTK_REQUIRE(w->a_p_w && w->a_g_w && w->b_p_w && w->b_g_w && w->g_w && w->z_w, GTK_EINVAL,
              "gtk_tri_mul_pack: null weight");
  const size_t need = gtk_tri_mul_packed_size(c_z, c, dtype);
  GTK_REQUIRE(packed_bytes >= need, GTK_EWORKSPACE, "gtk_tri_mul_pack: buffer %zu < %zu bytes",
              packed_bytes, need);
  hipStream_t st = (hipStream_t)stream;
  if (dtype == GTK_F32) return pack_trimul<float>(w, (int)c_z, (int)c, packed, st);
  return pack_trimul<bf16>(w, (int)c_z, (int)c, packed, st);
}

extern "C" size_t gtk_tri_mul_workspace_size_chunked(int64_t B, int64_t N, int64_t c_z, int64_t c,
                                                     int dtype, int64_t chunk_rows) {
  (void)c_z;
  if (B < 0 || N < 0 || c < 0 || chunk_rows < 0 || N > 16384) return 0;
  if (dtype != GTK_F32 && dtype != GTK_BF16) return 0;
  const int64_t Np = round_up(N, 64);
  const int64_t R = dtype == GTK_F32 ? trimul_chunk_rows<float>(N, chunk_rows)
                                     : trimul_chunk_rows<bf16>(N, chunk_rows);
  const size_t es = dtype_size(dtype);
  // plane_stride: each plane padded by 256 bytes
  return (size_t)(B * c) * ((size_t)(Np * Np) * es + 256) + 2 * (size_t)(B * c) * ((size_t)(R * Np) * es + 256) +
         3 * 256;
}

extern "C" size_t gtk_tri_mul_workspace_size(int64_t B, int64_t N, int64_t c_z, int64_t c, int dtype) {
  return gtk_tri_mul_workspace_size_chunked(B, N, c_z, c, dtype, 0);
}

extern "C" int gtk_tri_mul_forward_chunked(const void* z, const float* mask, void* out,
                                           const void* packed, int64_t B, int64_t N, int64_t c_z,
                                           int64_t c, int outgoing, int residual, float eps_in,
                                           float eps_out, int dtype, int64_t chunk_rows, void* ws,
                                           size_t ws_bytes, void* stream) {
  const char* name = chunk_rows ? "gtk_tri_mul_forward_chunked" : "gtk_tri_mul_forward";
  GTK_REQUIRE(dtype == GTK_F32 || dtype == GTK_BF16, GTK_EINVAL, "%s: bad dtype %d", name, dtype);
  GTK_REQUIRE(trimul_shape_ok(c_z, c), GTK_EUNSUPPORTED,
              "%s: c_z=%lld c=%lld unsupported (c_z in {32,64,128}, c in {32,64,128,256})", name,
              (long long)c_z, (long long)c);
  GTK_REQUIRE(B >= 0 && N >= 0 && N <= 16384, GTK_EINVAL, "%s: bad shape B=%lld N=%lld", name,
              (long long)B, (long long)N);
  GTK_REQUIRE(chunk_rows >= 0, GTK_EINVAL, "%s: chunk_rows=%lld < 0", name, (long long)chunk_rows);
  if (B == 0 || N == 0) return GTK_OK;
  GTK_REQUIRE(z && out && packed && ws, GTK_EINVAL, "%s: null pointer", name);
  const size_t need = gtk_tri_mul_workspace_size_chunked(B, N, c_z, c, dtype, chunk_rows);
  GTK_REQUIRE(ws_bytes >= need, GTK_EWORKSPACE, "%s: workspace %zu < %zu bytes", name, ws_bytes,
              need);
  hipStream_t st = (hipStream_t)stream;
  if (dtype == GTK_F32)
    return fwd_trimul_any<float>(c_z, c, z, mask, out, packed, B, N, outgoing, residual, eps_in,
                                 eps_out, ws, st, chunk_rows);
  return fwd_trimul_any<bf16>(c_z, c, z, mask, out, packed, B, N, outgoing, residual, eps_in,
                              eps_out, ws, st, chunk_rows);
}

extern "C" int gtk_tri_mul_forward(const void* z, const float* mask, void* out, const void* packed,
                                   int64_t B, int64_t N, int64_t c_z, int64_t c, int outgoing,
                                   int residual, float eps_in, float eps_out, int dtype, void* ws,
                                   size_t ws_bytes, void* stream) {
  return gtk_tri_mul_forward_chunked(z, mask, out, packed, B, N, c_z, c, outgoing, residual,
                                     eps_in, eps_out, dtype, 0, ws, ws_bytes, stream);
}

extern "C" size_t gtk_tri_mul_fp8ab_workspace_size(int64_t B, int64_t N, int64_t c_z, int64_t c) {
  if (B < 0 || N < 0 || N > 16384 || c_z != 128 || (c != 64 && c != 128)) return 0;
  const int64_t Np = fp8_np(N);
  // a, b (1 byte), x (2 bytes), each plane padded by 256 bytes (plane_stride)
  return (size_t)(B * c) * ((size_t)(Np * Np) * 4 + 3 * 256) + 3 * 256;
}

extern "C" int gtk_tri_mul_forward_fp8ab(const void* z, const float* mask, void* out,
                                         const void* packed, int64_t B, int64_t N, int64_t c_z,
                                         int64_t c, int outgoing, int residual, float eps_in,
                                         float eps_out, void* ws, size_t ws_bytes, void* stream) {
  GTK_REQUIRE(c_z == 128 && (c == 64 || c == 128), GTK_EUNSUPPORTED,
              "gtk_tri_mul_forward_fp8ab: c_z=%lld c=%lld unsupported (c_z 128, c in {64, 128})",
              (long long)c_z, (long long)c);
  GTK_REQUIRE(B >= 0 && N >= 0 && N <= 16384, GTK_EINVAL, "gtk_tri_mul_forward_fp8ab: bad shape");
  if (B == 0 || N == 0) return GTK_OK;
  GTK_REQUIRE(z && out && packed && ws, GTK_EINVAL, "gtk_tri_mul_forward_fp8ab: null pointer");
  const size_t need = gtk_tri_mul_fp8ab_workspace_size(B, N, c_z, c);
  GTK_REQUIRE(ws_bytes >= need, GTK_EWORKSPACE, "gtk_tri_mul_forward_fp8ab: workspace %zu < %zu bytes",
              ws_bytes, need);
  hipStream_t st = (hipStream_t)stream;
  if (c == 128)
    return fwd_trimul_fp8<128, 128>(z, mask, out, packed, B, N, outgoing, residual, eps_in, eps_out, ws, st);
  return fwd_trimul_fp8<128, 64>(z, mask, out, packed, B, N, outgoing, residual, eps_in, eps_out, ws, st);
}

extern "C" int gtk_tri_mul_contract_fp8(const void* a, const void* b, void* x, int64_t nplanes,
                                        int64_t Np, void* stream) {
  GTK_REQUIRE(nplanes >= 0 && Np >= 0 && Np % 256 == 0 && Np <= 16384, GTK_EINVAL,
              "gtk_tri_mul_contract_fp8: Np=%lld must be a multiple of 256 (<= 16384)", (long long)Np);
  if (nplanes == 0 || Np == 0) return GTK_OK;
  GTK_REQUIRE(a && b && x, GTK_EINVAL, "gtk_tri_mul_contract_fp8: null pointer");
  return launch_contract_fp8((const uint8_t*)a, (const uint8_t*)b, (bf16*)x, (int)Np, nplanes,
                             (hipStream_t)stream);
}
