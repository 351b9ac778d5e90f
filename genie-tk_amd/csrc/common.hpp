// Shared device-side building blocks for the gfx950 (CDNA4) pair-stack kernels.
//
// Conventions used by every kernel in this library
// -------------------------------------------------
// * A "row tile" is 32 pair rows handled by one wavefront (64 lanes).  Lane l
//   owns pair row (l & 31) and one half of that row's channels:
//   half = l >> 5 owns channels [half*C/2, half*C/2 + C/2).
// * Matrix-core work uses v_mfma_f32_32x32x16_bf16 (bf16 inputs) or
//   v_mfma_f32_32x32x2_f32 (fp32 inputs), always with fp32 accumulation.
//   Both instructions take, per lane, operand values for ONE row (A) or ONE
//   column (B) indexed by (l & 31), and a k-group selected by (l >> 5).
//   Because A and B use the same lane->k assignment, any bijection between
//   "k-slot" and real contraction index is valid as long as both operands use
//   it.  We use: chunk ks, lane half h, element e  <->  k = h*K/2 + ks*8 + e,
//   so every lane reads 8 *consecutive* channels (16 B of bf16) per chunk.
// * Accumulator layout of a 32x32 MFMA tile (16 fp32 per lane):
//   acc[4*g + r]  <->  row 8*g + 4*(l>>5) + r,  column (l & 31).
// * bf16 is stored as the compiler's native __bf16; fp32 -> bf16 conversion
//   is round-to-nearest-even (v_cvt_pk_bf16_f32 on gfx950).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace gtk {

typedef __bf16 bf16;
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));

constexpr float kLog2e = 1.4426950408889634f;

// ---------------------------------------------------------------------------
// 8-element fragments: the per-lane operand of one 16-wide k chunk.
// ---------------------------------------------------------------------------
template <typename T> struct Frag;

template <> struct Frag<bf16> {
  bf16x8 v;
  __device__ __forceinline__ void load(const bf16* p) { v = *reinterpret_cast<const bf16x8*>(p); }
  __device__ __forceinline__ void zero() {
    for (int e = 0; e < 8; ++e) v[e] = (bf16)0.0f;
  }
  __device__ __forceinline__ void set(const float* f) {
    for (int e = 0; e < 8; ++e) v[e] = (bf16)f[e];
  }
  __device__ __forceinline__ float get(int e) const { return (float)v[e]; }
};

template <> struct Frag<float> {
  f32x4 lo, hi;
  __device__ __forceinline__ void load(const float* p) {
    lo = *reinterpret_cast<const f32x4*>(p);
    hi = *reinterpret_cast<const f32x4*>(p + 4);
  }
  __device__ __forceinline__ void zero() {
    lo = f32x4{0.f, 0.f, 0.f, 0.f};
    hi = lo;
  }
  __device__ __forceinline__ void set(const float* f) {
    for (int e = 0; e < 4; ++e) { lo[e] = f[e]; hi[e] = f[e + 4]; }
  }
  __device__ __forceinline__ float get(int e) const { return e < 4 ? lo[e] : hi[e - 4]; }
};

// acc += A(32x16 chunk) * B(16x32 chunk)
__device__ __forceinline__ void mma(f32x16& acc, const Frag<bf16>& a, const Frag<bf16>& b) {
  acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a.v, b.v, acc, 0, 0, 0);
}
__device__ __forceinline__ void mma(f32x16& acc, const Frag<float>& a, const Frag<float>& b) {
  for (int e = 0; e < 4; ++e) acc = __builtin_amdgcn_mfma_f32_32x32x2f32(a.lo[e], b.lo[e], acc, 0, 0, 0);
  for (int e = 0; e < 4; ++e) acc = __builtin_amdgcn_mfma_f32_32x32x2f32(a.hi[e], b.hi[e], acc, 0, 0, 0);
}

// This wave's index in its block, as a wave-uniform value (readfirstlane):
// index math derived from it stays in scalar registers, and buffer
// resources built from it need no per-lane waterfall loop.
__device__ __forceinline__ int wave_id() { return __builtin_amdgcn_readfirstlane(threadIdx.x >> 6); }

__device__ __forceinline__ f32x16 zero16() {
  f32x16 z;
  for (int e = 0; e < 16; ++e) z[e] = 0.f;
  return z;
}

// ---------------------------------------------------------------------------
// Scalar conversions and small vector stores.
// ---------------------------------------------------------------------------
template <typename T> __device__ __forceinline__ T cvt(float f);
template <> __device__ __forceinline__ float cvt<float>(float f) { return f; }
template <> __device__ __forceinline__ bf16 cvt<bf16>(float f) { return (bf16)f; }

__device__ __forceinline__ float to_f32(float x) { return x; }
__device__ __forceinline__ float to_f32(bf16 x) { return (float)x; }

// Store 4 consecutive values.
__device__ __forceinline__ void store4(bf16* p, float a, float b, float c, float d) {
  bf16x4 v;
  v[0] = (bf16)a; v[1] = (bf16)b; v[2] = (bf16)c; v[3] = (bf16)d;
  *reinterpret_cast<bf16x4*>(p) = v;
}
__device__ __forceinline__ void store4(float* p, float a, float b, float c, float d) {
  *reinterpret_cast<f32x4*>(p) = f32x4{a, b, c, d};
}
// Two values as packed bf16 (low half = a).
__device__ __forceinline__ uint32_t pack_bf16x2(float a, float b) {
  typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
  bf16x2 v;
  v[0] = (bf16)a;
  v[1] = (bf16)b;
  return __builtin_bit_cast(uint32_t, v);
}
// Raw buffer resource over `bytes` bytes at `base`.  A buffer access whose
// offset is >= bytes does nothing (a store is dropped): lanes without a valid
// destination pass kBufSkip instead of branching around the store, so every
// lane runs the same instruction stream (and the compiler's wait counts see
// one path).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t buf_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, 0x00020000);
}
// buf_rsrc for a base the caller knows is wave-uniform but the compiler may
// not (64-bit address arithmetic it did on the VALU): both halves go through
// readfirstlane, so the descriptor lands in SGPRs and no buffer access needs
// a waterfall loop.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t buf_rsrc_u(const void* base, uint32_t bytes) {
  const uint64_t a = (uint64_t)(uintptr_t)base;
  const uint64_t u = ((uint64_t)(uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)(a >> 32)) << 32) |
                     (uint64_t)(uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)a);
  return buf_rsrc(reinterpret_cast<const void*>(u), bytes);
}
constexpr uint32_t kBufSkip = 0x80000000u;
// 4 values as bf16 (8 bytes) at byte offset `off`.
__device__ __forceinline__ void buf_store4(__amdgpu_buffer_rsrc_t r, uint32_t off, float a, float b,
                                           float c, float d) {
  typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
  const u32x2 v = {pack_bf16x2(a, b), pack_bf16x2(c, d)};
  __builtin_amdgcn_raw_buffer_store_b64(v, r, off, 0, 0);
}

// 16 bytes at byte offset `off` (same range rule as buf_store4).
__device__ __forceinline__ void buf_store16(__amdgpu_buffer_rsrc_t r, uint32_t off, uint4 v) {
  typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
  __builtin_amdgcn_raw_buffer_store_b128(u32x4{v.x, v.y, v.z, v.w}, r, off, 0, 0);
}

// Cache policy of a buffer store: device scope (sc1).  The store writes
// through the XCD's L2 instead of leaving the line dirty there; for a kernel
// that streams its output once (LayerNorm over the pair tensor) this was
// 3-11 % faster than a plain store on MI355X, measured together with
// non-temporal loads.
constexpr int kStoreSc1 = 16;
// 16 bytes at byte offset `off` with the device-scope policy (same range rule
// as buf_store4).
__device__ __forceinline__ void buf_store16_sc1(__amdgpu_buffer_rsrc_t r, uint32_t off, uint4 v) {
  typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
  __builtin_amdgcn_raw_buffer_store_b128(u32x4{v.x, v.y, v.z, v.w}, r, off, 0, kStoreSc1);
}
// 16 bytes with the non-temporal hint (data read once).
__device__ __forceinline__ uint4 load16_nt(const void* p) {
  typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
  const u32x4 v = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
  return uint4{v.x, v.y, v.z, v.w};
}

// Load 4 consecutive values as fp32.
__device__ __forceinline__ f32x4 load4f(const bf16* p) {
  bf16x4 v = *reinterpret_cast<const bf16x4*>(p);
  return f32x4{(float)v[0], (float)v[1], (float)v[2], (float)v[3]};
}
__device__ __forceinline__ f32x4 load4f(const float* p) { return *reinterpret_cast<const f32x4*>(p); }

__device__ __forceinline__ float sigmoidf_(float x) { return 1.0f / (1.0f + __expf(-x)); }

// Value held by lane (l ^ 32).
__device__ __forceinline__ float xor32(float v) { return __shfl_xor(v, 32, 64); }

// ---------------------------------------------------------------------------
// Row-tile LayerNorm in fragment layout.
//
// Lane l holds pair row (l & 31), channels half*C/2 + [0, C/2) as C/16
// fragments of 8.  The row statistics combine the lane's own half with lane
// (l ^ 32)'s half.  Two-pass (mean, then centred sum of squares), biased
// variance, eps inside the square root: x_hat = (x - mu) / sqrt(var + eps).
// The LayerNorm weight w and bias b never reach the kernels: a LayerNorm
// followed by a linear map W, c is computed as (W diag(w)) x_hat + (W b + c),
// with both terms prepared when the weights are packed.
// ---------------------------------------------------------------------------
template <int C> struct RowHalf {
  static constexpr int NCH = C / 16;  // fragments per lane
  float v[C / 2];
};

template <typename TIn, int C>
__device__ __forceinline__ void load_row_half(RowHalf<C>& r, const TIn* row_base, bool valid) {
  const int half = (threadIdx.x & 63) >> 5;
  const TIn* p = row_base + half * (C / 2);
  if (valid) {
#pragma unroll
    for (int ch = 0; ch < C / 16; ++ch) {
      Frag<TIn> f;
      f.load(p + ch * 8);
#pragma unroll
      for (int e = 0; e < 8; ++e) r.v[ch * 8 + e] = f.get(e);
    }
  } else {
#pragma unroll
    for (int i = 0; i < C / 2; ++i) r.v[i] = 0.f;
  }
}

// Returns (mean, rstd) of the full row of C channels.
template <int C>
__device__ __forceinline__ f32x2 row_stats(const RowHalf<C>& r, float eps) {
  float s = 0.f;
#pragma unroll
  for (int i = 0; i < C / 2; ++i) s += r.v[i];
  s += xor32(s);
  const float mean = s * (1.0f / C);
  float q = 0.f;
#pragma unroll
  for (int i = 0; i < C / 2; ++i) {
    const float d = r.v[i] - mean;
    q += d * d;
  }
  q += xor32(q);
  const float var = q * (1.0f / C);
  return f32x2{mean, __builtin_amdgcn_rsqf(var + eps)};  // v_rsq_f32 (1 ulp)
}

// Normalise (no affine: the LayerNorm weight and bias are folded into the
// packed weights of the linear map that follows), then pack into fragments.
template <typename T, int C>
__device__ __forceinline__ void ln_to_frags(Frag<T>* frags, const RowHalf<C>& r, f32x2 st) {
#pragma unroll
  for (int ch = 0; ch < C / 16; ++ch) {
    float f[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) f[e] = (r.v[ch * 8 + e] - st[0]) * st[1];
    frags[ch].set(f);
  }
}

// Normalise and apply the LayerNorm affine (gamma, beta: fp32 [C]) before the
// conversion to the fragment type: one rounding of the LayerNorm output, for
// linear maps packed without the affine folded in.
template <typename T, int C>
__device__ __forceinline__ void ln_affine_to_frags(Frag<T>* frags, const RowHalf<C>& r, f32x2 st,
                                                   const float* __restrict__ gamma,
                                                   const float* __restrict__ beta) {
  const int c0 = ((threadIdx.x & 63) >> 5) * (C / 2);  // this lane's channel half
#pragma unroll
  for (int ch = 0; ch < C / 16; ++ch) {
    float f[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const int c = c0 + ch * 8 + e;
      f[e] = (r.v[ch * 8 + e] - st[0]) * st[1] * gamma[c] + beta[c];
    }
    frags[ch].set(f);
  }
}

// Row-tile LayerNorm (normalise only) straight from bf16 storage into bf16
// fragments: the raw
// half row stays packed (C/4 VGPRs) and is widened on the fly, so the peak
// register footprint is two sets of packed fragments.
// LayerNorm (normalisation only) of the pair row held as raw bf16 fragments:
// lane l holds channels (l>>5)*C/2 + 8*ch + e of its row in raw[ch]; the two
// lanes of a row exchange partial sums with one lane^32 swap.
template <int C>
__device__ __forceinline__ void ln_frags_bf16(Frag<bf16>* xf, const Frag<bf16>* raw, float eps) {
  float s = 0.f;
#pragma unroll
  for (int ch = 0; ch < C / 16; ++ch)
#pragma unroll
    for (int e = 0; e < 8; ++e) s += raw[ch].get(e);
  s += xor32(s);
  const float mean = s * (1.0f / C);
  float q = 0.f;
#pragma unroll
  for (int ch = 0; ch < C / 16; ++ch)
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float d = raw[ch].get(e) - mean;
      q += d * d;
    }
  q += xor32(q);
  const float rstd = __builtin_amdgcn_rsqf(q * (1.0f / C) + eps);  // v_rsq_f32 (1 ulp)
#pragma unroll
  for (int ch = 0; ch < C / 16; ++ch) {
    float f[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) f[e] = (raw[ch].get(e) - mean) * rstd;
    xf[ch].set(f);
  }
}

// Load and normalise the pair row at row_base (zeros when !valid).
template <int C>
__device__ __forceinline__ void ln_row_bf16(Frag<bf16>* xf, const bf16* row_base, bool valid,
                                            float eps) {
  const int half = (threadIdx.x & 63) >> 5;
  Frag<bf16> raw[C / 16];
#pragma unroll
  for (int ch = 0; ch < C / 16; ++ch) {
    if (valid) raw[ch].load(row_base + half * (C / 2) + ch * 8);
    else raw[ch].zero();
  }
  ln_frags_bf16<C>(xf, raw, eps);
}

// Transposing LDS read (ds_read_b64_tr_b16).  Within each group of 16 lanes,
// lane L receives element L%4 of the 4 elements read at the addresses of
// lanes L/4, 4 + L/4, 8 + L/4 and 12 + L/4 (in that order).
typedef short s16x4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ s16x4 lds_read_tr16(const void* p) {
  return __builtin_amdgcn_ds_read_tr16_b64_v4i16(
      (__attribute__((address_space(3))) s16x4*)(const_cast<void*>(p)));
}

// ---------------------------------------------------------------------------
// Packed weight fragments.
//
// A Linear weight W[out][in] (nn.Linear layout) is packed for K = in so that
// fragment (tile nt, chunk ks) is 64 lanes x 8 contiguous elements:
//   packed[((nt*KCH + ks)*64 + l)*8 + e] = W[nt*32 + (l&31)][(l>>5)*K/2 + ks*8 + e]
// (zero for out >= OUT).  One wave reads a fragment as 1 KiB (bf16) contiguous.
// ---------------------------------------------------------------------------
template <typename T>
__device__ __forceinline__ void load_wfrag(Frag<T>& f, const T* __restrict__ packed, int nt, int ks, int kch) {
  const int l = threadIdx.x & 63;
  f.load(packed + ((size_t)(nt * kch + ks) * 64 + l) * 8);
}

// Same fragment from a packed weight copy resident in LDS (64 lanes read
// 1 KiB contiguous: bank-conflict free).
__device__ __forceinline__ void load_wfrag_lds(Frag<bf16>& f, const bf16* packed_lds, int nt, int ks,
                                               int kch) {
  const int l = threadIdx.x & 63;
  f.load(packed_lds + ((nt * kch + ks) * 64 + l) * 8);
}

typedef __attribute__((address_space(3))) void* lds_void_ptr;

// 16 bytes per lane from global memory straight into LDS at
// (wave-uniform base) + lane * 16 (global_load_lds_dwordx4, no VGPR staging).
//
// Issued from inline asm on purpose.  Through the compiler builtin, the
// waitcnt pass cannot tell which LDS bytes the copy writes, so it puts an
// s_waitcnt vmcnt(0) before the next LDS read of ANY address: a copy of the
// next pipeline stage then completes before the current stage is read, and
// copies never overlap compute.  Hidden from that pass, the copy is ordered
// only by the caller's explicit s_waitcnt vmcnt(n) (vmcnt counts every
// vector-memory load in issue order, these included) followed by a block
// barrier, or by __syncthreads(), whose fence waits for vmcnt(0).  M0 (the
// copy's LDS base) is a reserved register: the asm restores it.
__device__ __forceinline__ void g2lds16(const void* gptr, void* lds_wave_base) {
  const uint32_t lds = __builtin_amdgcn_readfirstlane(
      (uint32_t)(uintptr_t)(lds_void_ptr)lds_wave_base);
  uint32_t saved;
  asm volatile(
      "s_mov_b32 %0, m0\n\t"
      "s_mov_b32 m0, %2\n\t"
      "s_nop 0\n\t"
      "global_load_lds_dwordx4 %1, off\n\t"
      "s_mov_b32 m0, %0"
      : "=&s"(saved)
      : "v"(gptr), "s"(lds)
      : "memory");
}

// 4 bytes per lane from global memory into LDS at (wave-uniform base) +
// lane * 4: used to pull lines into L2 ahead of their real copies (the LDS
// bytes are a scratch area nobody reads, and no VGPR is written, so nothing
// depends on when the load lands).  Same ordering contract as g2lds16.
__device__ __forceinline__ void g2lds4(const void* gptr, uint32_t lds) {
  uint32_t saved;
  asm volatile(
      "s_mov_b32 %0, m0\n\t"
      "s_mov_b32 m0, %2\n\t"
      "s_nop 0\n\t"
      "global_load_lds_dword %1, off\n\t"
      "s_mov_b32 m0, %0"
      : "=&s"(saved)
      : "v"(gptr), "s"(lds)
      : "memory");
}

// LDS byte address of a __shared__ object, for the copies below.
__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)(lds_void_ptr)p);
}

// g2lds16 with a wave-uniform 64-bit base in scalar registers and a 32-bit
// per-lane byte offset (the saddr form: one VGPR per copy instead of two);
// `lds` is the wave's LDS destination address (lds_addr).  Same ordering
// contract as g2lds16.
__device__ __forceinline__ void g2lds16_sv(const void* sbase, uint32_t voff, uint32_t lds) {
  uint32_t saved;
  asm volatile(
      "s_mov_b32 %0, m0\n\t"
      "s_mov_b32 m0, %3\n\t"
      "s_nop 0\n\t"
      "global_load_lds_dwordx4 %1, %2\n\t"
      "s_mov_b32 m0, %0"
      : "=&s"(saved)
      : "v"(voff), "s"(sbase), "s"(lds)
      : "memory");
}

// g2lds16_sv for data read once (the non-temporal hint): the copy is streamed
// through the caches with low retention, so it does not evict data that other
// waves re-read from L2.
__device__ __forceinline__ void g2lds16_sv_nt(const void* sbase, uint32_t voff, uint32_t lds) {
  uint32_t saved;
  asm volatile(
      "s_mov_b32 %0, m0\n\t"
      "s_mov_b32 m0, %3\n\t"
      "s_nop 0\n\t"
      "global_load_lds_dwordx4 %1, %2 nt\n\t"
      "s_mov_b32 m0, %0"
      : "=&s"(saved)
      : "v"(voff), "s"(sbase), "s"(lds)
      : "memory");
}

// Asynchronously copy `bytes` (a multiple of 1 KiB) from global memory into
// LDS with the whole block: every load is issued before any is waited for.
// The caller waits (s_waitcnt vmcnt(0)) and synchronises the block.
__device__ __forceinline__ void copy_to_lds_async(void* dst, const void* __restrict__ src, int bytes) {
  const int lane = threadIdx.x & 63;
  const int wave = wave_id();
  const int nwaves = blockDim.x >> 6;
  for (int blk = wave; blk * 1024 < bytes; blk += nwaves)
    g2lds16((const char*)src + blk * 1024 + lane * 16, (char*)dst + blk * 1024);
}

// A linear tile index t = (b * rows + r) * cols + c, walked by a fixed stride
// without divisions: a 64-bit division by a run-time value costs tens of
// instructions, per tile, in the persistent loops.  Divides once at set-up.
struct TileWalk {
  int b, r, c;     // the current tile
  int db, dr, dc;  // the stride, decomposed the same way
  int rows, cols;
  __device__ __forceinline__ void init(int64_t t, int64_t stride, int rows_, int cols_) {
    rows = rows_;
    cols = cols_;
    const int64_t plane = (int64_t)rows * cols;
    c = (int)(t % cols);
    r = (int)((t / cols) % rows);
    b = (int)(t / plane);
    dc = (int)(stride % cols);
    dr = (int)((stride / cols) % rows);
    db = (int)(stride / plane);
  }
  __device__ __forceinline__ void next() {
    c += dc;
    int carry = 0;
    if (c >= cols) {
      c -= cols;
      carry = 1;
    }
    r += dr + carry;  // < 2 * rows
    if (r >= rows) {
      r -= rows;
      b += 1;
    }
    b += db;
  }
};

// s_waitcnt immediate for vmcnt(N) alone (expcnt and lgkmcnt not waited for);
// vmcnt is 6 bits on gfx950: [3:0] and [15:14].
template <int N>
constexpr int vmcnt_imm() {
  static_assert(N >= 0 && N < 64, "vmcnt is 6 bits");
  return 0x0F70 | (N & 15) | ((N >> 4) << 14);
}

// s_barrier without the fence that __syncthreads() adds: that fence waits for
// every outstanding global load, including direct-to-LDS copies meant to stay
// in flight across the barrier.  Callers order memory themselves with
// explicit s_waitcnt; the "memory" clobber keeps the compiler from moving
// memory accesses across the barrier.  The lgkmcnt(0) makes this wave's LDS
// reads complete first, so a copy issued after the barrier into a stage the
// waves just read cannot overtake a read still in flight.
__device__ __forceinline__ void barrier_only() {
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

// XCD-aware block order: hardware deals consecutive block ids to the 8 XCDs
// round-robin; remap so that each XCD receives a contiguous range of logical
// blocks (blocks that share operands then share that XCD's L2).
__device__ __forceinline__ int64_t xcd_remap(int64_t lin, int64_t total) {
  if (total % 8 != 0) return lin;
  return (lin % 8) * (total / 8) + lin / 8;
}

// A zero the compiler cannot see through.  Adding it to a loop-invariant LDS
// address inside a loop keeps the loads in the loop: hoisted out, the
// fragments would stay live across the whole loop and spill.
__device__ __forceinline__ int opaque_zero() {
  int z;
  asm volatile("v_mov_b32 %0, 0" : "=v"(z));
  return z;
}

// acc = A . B with a zero accumulator input (inline constant, no register init).
__device__ __forceinline__ f32x16 mma0(const Frag<bf16>& a, const Frag<bf16>& b) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a.v, b.v, zero16(), 0, 0, 0);
}

// sigmoid(x) for u = -x * log2(e) (gate projections are packed pre-scaled):
// 1 / (1 + 2^u) with the hardware reciprocal.
__device__ __forceinline__ float gate_from_u(float u) {
  return __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(u));
}

// acc(32 pairs x 32 outputs of tile nt) = rows . W_nt^T over K = C.
// SWAP=false: acc rows = pairs, cols = outputs.  SWAP=true: rows = outputs, cols = pairs.
template <typename T, int C, bool SWAP>
__device__ __forceinline__ f32x16 row_gemm_tile(const Frag<T>* xf, const T* __restrict__ packed, int nt) {
  f32x16 acc = zero16();
#pragma unroll
  for (int ks = 0; ks < C / 16; ++ks) {
    Frag<T> w;
    load_wfrag<T>(w, packed, nt, ks, C / 16);
    if (SWAP) mma(acc, w, xf[ks]);
    else mma(acc, xf[ks], w);
  }
  return acc;
}

}  // namespace gtk
