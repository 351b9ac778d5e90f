// Declarations shared by the triangle-multiplication forward (tri_mul.hip)
// and backward (tri_mul_bwd.hip).
#pragma once
#include "capi_util.hpp"
#include "common.hpp"
#include "pack.hpp"

namespace gtk {

// Packed parameters of one TriangleMultiplicativeUpdate, carved in this order.
// For the shapes with backward kernels (c_z = 128, c in {64, 128}) the weights
// carry the LayerNorm weights folded in (w_ap..w_g: layer_norm_in, w_z:
// layer_norm_out) and the biases the LayerNorm biases (b = W beta + c); the
// other shapes keep the plain weights and biases, and their kernels apply the
// LayerNorm affine from the fp32 copies ln_* before rounding the normalised
// row once (one bf16 rounding instead of two for the small channel counts).
template <int CZ, int CH>
constexpr bool trimul_folded() {
  return CZ == 128 && (CH == 64 || CH == 128);
}
inline bool trimul_folded_rt(int cz, int c) { return cz == 128 && (c == 64 || c == 128); }

template <typename T> struct TriMulPacked {
  T *w_ap, *w_ag, *w_bp, *w_bg, *w_g, *w_z;
  float *b_ap, *b_ag, *b_bp, *b_bg, *b_g, *b_z;
  float *ln_in_w, *ln_in_b, *ln_out_w, *ln_out_b;
};

template <typename T>
static TriMulPacked<T> carve_trimul(Carve& cv, int cz, int c) {
  TriMulPacked<T> p;
  p.w_ap = cv.take<T>(packed_elems(c, cz));
  p.w_ag = cv.take<T>(packed_elems(c, cz));
  p.w_bp = cv.take<T>(packed_elems(c, cz));
  p.w_bg = cv.take<T>(packed_elems(c, cz));
  p.w_g = cv.take<T>(packed_elems(cz, cz));
  p.w_z = cv.take<T>(packed_elems(cz, c));
  p.b_ap = cv.take<float>(c);
  p.b_ag = cv.take<float>(c);
  p.b_bp = cv.take<float>(c);
  p.b_bg = cv.take<float>(c);
  p.b_g = cv.take<float>(cz);
  p.b_z = cv.take<float>(cz);
  p.ln_in_w = cv.take<float>(cz);
  p.ln_in_b = cv.take<float>(cz);
  p.ln_out_w = cv.take<float>(c);
  p.ln_out_b = cv.take<float>(c);
  return p;
}

// Forward pieces the backward re-runs (defined in tri_mul.hip):
// the A and Bm planes of the prologue and X = A Bm^T, into caller buffers of
// B*c planes [Np][Np] each (Np = N rounded up to 64).
int trimul_recompute_planes(const void* z, const float* mask, const void* packed, int64_t B,
                            int64_t N, int64_t c_z, int64_t c, int outgoing, float eps_in,
                            int dtype, void* pa, void* pb, void* px, hipStream_t st);
// out = L R^T per [Np][Np] plane (nplanes planes).
int trimul_contract_planes(const void* pl, const void* pr, void* out, int Np, int64_t nplanes,
                           int dtype, hipStream_t st);
// The same with L given as the plane L^T (lt) and / or R as R^T (rt):
// bf16 planes whose contraction takes the 256 or 128 tile kernels
// (trimul_contract_t_ok); elsewhere the caller transposes the planes.
bool trimul_contract_t_ok(int Np, int64_t nplanes, int dtype);
int trimul_contract_planes_t(const void* pl, const void* pr, void* out, int Np, int64_t nplanes, bool lt,
                             bool rt, hipStream_t st);

}  // namespace gtk
