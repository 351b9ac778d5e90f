/*
 * genie_tk.h — C ABI of the MI355X (gfx950) pair-stack kernels.
 *
 * Every function takes device pointers, plain sizes and a HIP stream passed
 * as `void*` (a hipStream_t; NULL means the legacy default stream).  No
 * function allocates device memory: scratch space is passed in by the caller
 * as (workspace, workspace_bytes), sized with the matching *_workspace_size()
 * query.  Every function enqueues work on `stream` and returns without
 * synchronising.  Return value: GTK_OK (0) or a GTK_E* code; the message of
 * the last failure on the calling thread is returned by gtk_last_error().
 *
 * Element types: GTK_F32 (float) and GTK_BF16 (bfloat16, round-to-nearest-even
 * on every conversion).  bf16 inputs are contracted on the bf16 matrix cores
 * with fp32 accumulation; fp32 inputs use the fp32 matrix cores.
 *
 * Layouts (row-major, innermost last):
 *   pair tensor z / x        [B][N][N][C]
 *   pair mask                [B][N][N]   float, 1 = valid, 0 = masked
 *   nn.Linear weight         [out][in]
 *
 * The reference interface each entry point replaces is cited as
 * path:line in the upstream Genie-TK repository.
 */
#ifndef GENIE_TK_H_
#define GENIE_TK_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum gtk_dtype { GTK_F32 = 0, GTK_BF16 = 1 };

enum gtk_status {
  GTK_OK = 0,
  GTK_EINVAL = 1,       /* bad pointer, size or dtype */
  GTK_EUNSUPPORTED = 2, /* a shape the kernels are not built for */
  GTK_EWORKSPACE = 3,   /* workspace / packed buffer too small */
  GTK_EHIP = 4          /* a HIP runtime call or launch failed */
};

/* Message of the last error on this thread ("" if none). */
const char* gtk_last_error(void);
/* Library version: major*10000 + minor*100 + patch. */
int gtk_version(void);

/* ------------------------------------------------------------------------
 * LayerNorm over the last dimension.
 * Replaces _C.layernorm(x, gamma, beta, eps)
 *   kernels/bindings.cpp:93-95 -> kernels/fused_layernorm/layernorm.cu:17-44.
 * y = (x - mean) / sqrt(var_biased + eps) * gamma + beta, per row of d.
 * x, y: [rows][d] of `dtype`; gamma, beta: [d] float.  y may not alias x.
 * ------------------------------------------------------------------------ */
int gtk_layernorm(const void* x, void* y, const float* gamma, const float* beta, int64_t rows,
                  int64_t d, float eps, int dtype, void* stream);

/* ------------------------------------------------------------------------
 * LayerNorm followed by a linear map.
 * Replaces _C.fused_layernorm_linear(x, gamma, beta, weight, bias, eps)
 *   kernels/bindings.cpp:97-100 -> kernels/fused_layernorm/layernorm.cu:46-79.
 * y[r][o] = sum_k LN(x)[r][k] * weight[k][o] + bias[o]
 * weight: [d_in][d_out] (in x out, as the reference) of `weight_dtype`;
 * bias: [d_out] float or NULL.  d_in in {64, 128, 256}; any d_out >= 1.
 * ------------------------------------------------------------------------ */
size_t gtk_fused_layernorm_linear_workspace_size(int64_t d_in, int64_t d_out, int dtype);
int gtk_fused_layernorm_linear(const void* x, void* y, const float* gamma, const float* beta,
                               const void* weight, int weight_dtype, const float* bias,
                               int64_t rows, int64_t d_in, int64_t d_out, float eps, int dtype,
                               void* workspace, size_t workspace_bytes, void* stream);

/* The same operator with the weight in either layout: GTK_W_IN_OUT is
 * [d_in][d_out] (the reference's _C.fused_layernorm_linear), GTK_W_OUT_IN is
 * [d_out][d_in] (torch.nn.Linear.weight).  The generalisation of the
 * reference's operator to nn.Linear-layout weights has no reference
 * counterpart; the arithmetic is the one above.  Same workspace size. */
enum gtk_weight_layout { GTK_W_IN_OUT = 0, GTK_W_OUT_IN = 1 };
int gtk_layernorm_linear(const void* x, void* y, const float* gamma, const float* beta,
                         const void* weight, int weight_dtype, int weight_layout,
                         const float* bias, int64_t rows, int64_t d_in, int64_t d_out, float eps,
                         int dtype, void* workspace, size_t workspace_bytes, void* stream);

/* No-allocation form of gtk_layernorm_linear, for callers that cannot
 * allocate device memory or pass a workspace (code under HIP graph capture,
 * tight serving loops, harnesses that forbid allocation).  It has no
 * counterpart in the reference.  The scratch (the packed weight and the
 * folded bias) lives in a static device array of
 * GTK_LAYERNORM_LINEAR_SCRATCH_BYTES that each GPU holds until the process
 * ends; shapes whose gtk_fused_layernorm_linear_workspace_size exceeds it are
 * rejected with GTK_EWORKSPACE (bf16: d_in=128 up to d_out=4032, d_in=256 up
 * to d_out=2016).  The call allocates nothing.  All calls on one GPU share
 * the array: calls that overlap on one GPU (other streams or threads) race;
 * calls on one stream are ordered.  Same arguments and result as
 * gtk_layernorm_linear. */
#define GTK_LAYERNORM_LINEAR_SCRATCH_BYTES (1u << 20)
int gtk_layernorm_linear_noalloc(const void* x, void* y, const float* gamma, const float* beta,
                                 const void* weight, int weight_dtype, int weight_layout,
                                 const float* bias, int64_t rows, int64_t d_in, int64_t d_out,
                                 float eps, int dtype, void* stream);

/* ------------------------------------------------------------------------
 * Triangle contraction on already gated and masked projections.
 * Replaces _C.triangle_mul_outgoing / _C.triangle_mul_incoming(a, b, mask)
 *   kernels/bindings.cpp:73-79 (declared at :16-26); caller
 *   src/genie_tk/triangle_mul.py:151-159.
 * outgoing: x[b][i][j][c] = sum_k a[b][i][k][c] * b[b][j][k][c]
 * incoming: x[b][i][j][c] = sum_k a[b][k][i][c] * b[b][k][j][c]
 * a, b, x: [B][N][N][C] of `dtype`.  `mask` ([B][N][N] float) is accepted for
 * signature compatibility and not read: a and b arrive masked.
 * C % 16 == 0, N <= 16384.
 * ------------------------------------------------------------------------ */
size_t gtk_triangle_mul_workspace_size(int64_t B, int64_t N, int64_t C, int dtype);
int gtk_triangle_mul_outgoing(const void* a, const void* b, const float* mask, void* x, int64_t B,
                              int64_t N, int64_t C, int dtype, void* workspace,
                              size_t workspace_bytes, void* stream);
int gtk_triangle_mul_incoming(const void* a, const void* b, const float* mask, void* x, int64_t B,
                              int64_t N, int64_t C, int dtype, void* workspace,
                              size_t workspace_bytes, void* stream);

/* ------------------------------------------------------------------------
 * Triangle attention core on projected q, k, v.
 * Replaces _C.triangle_attention_starting / _ending(q, k, v, bias, mask, scale)
 *   kernels/bindings.cpp:82-90 (declared at :29-47).
 * q, k, v: [B][H][N][N][D] of `dtype`; bias: [B][H][N][N] float; mask:
 * [B][N][N] float; out: [B][N][N][H*D] of `dtype`.
 * starting (attention along the second spatial axis, rows i independent):
 *   out[b][i][q][h*D+d] = sum_k softmax_k(scale*<q[b,h,i,q], k[b,h,i,k]>
 *                              + mask_bias[b,i,k] + bias[b,h,q,k]) * v[b,h,i,k,d]
 * ending (attention along the first spatial axis, columns j independent):
 *   out[b][q][j][h*D+d] = sum_k softmax_k(scale*<q[b,h,q,j], k[b,h,k,j]>
 *                              + mask_bias[b,k,j] + bias[b,h,q,k]) * v[b,h,k,j,d]
 * mask_bias = 1e9 * (mask - 1), the additive bias of the reference's
 * TriangleAttention with its default inf = 1e9 (triangle_attention.py:57,118),
 * in fp32: a masked key takes no weight in a row with a valid key, and a row
 * whose keys are all masked (mask = 0) attends uniformly, as every score of
 * such a row rounds to -1e9 in fp32.  D == 32, N <= 8192.
 * ------------------------------------------------------------------------ */
size_t gtk_triangle_attention_workspace_size(int64_t B, int64_t H, int64_t N, int64_t D, int dtype);
int gtk_triangle_attention_starting(const void* q, const void* k, const void* v, const float* bias,
                                    const float* mask, float scale, void* out, int64_t B,
                                    int64_t H, int64_t N, int64_t D, int dtype, void* workspace,
                                    size_t workspace_bytes, void* stream);
int gtk_triangle_attention_ending(const void* q, const void* k, const void* v, const float* bias,
                                  const float* mask, float scale, void* out, int64_t B, int64_t H,
                                  int64_t N, int64_t D, int dtype, void* workspace,
                                  size_t workspace_bytes, void* stream);

/* ------------------------------------------------------------------------
 * Fused TriangleMultiplicativeUpdate forward (outgoing / incoming).
 * Replaces TriangleMultiplicativeUpdate._forward_cuda
 *   src/genie_tk/triangle_mul.py:134-169 (semantics of _forward_pytorch :103-132):
 *   zn  = LN_in(z)
 *   a   = (zn W_ap^T + b_ap) * sigmoid(zn W_ag^T + b_ag) * mask
 *   b   = (zn W_bp^T + b_bp) * sigmoid(zn W_bg^T + b_bg) * mask
 *   x   = outgoing ? einsum(bikc,bjkc->bijc) : einsum(bkic,bkjc->bijc)
 *   out = (LN_out(x) W_z^T + b_z) * sigmoid(zn W_g^T + b_g)   [+ z if residual]
 * Weights are first packed once with gtk_tri_mul_pack (the packed buffer
 * stays valid until the parameters change).  c_z in {32, 64, 128},
 * c in {32, 64, 128, 256},
 * N <= 16384.
 * ------------------------------------------------------------------------ */
typedef struct gtk_tri_mul_weights {
  int dtype;                     /* element type of every pointer below */
  const void *ln_in_w, *ln_in_b; /* [c_z]            layer_norm_in   */
  const void *a_p_w, *a_p_b;     /* [c][c_z], [c]    linear_a_p      */
  const void *a_g_w, *a_g_b;     /* [c][c_z], [c]    linear_a_g      */
  const void *b_p_w, *b_p_b;     /* [c][c_z], [c]    linear_b_p      */
  const void *b_g_w, *b_g_b;     /* [c][c_z], [c]    linear_b_g      */
  const void *g_w, *g_b;         /* [c_z][c_z],[c_z] linear_g        */
  const void *ln_out_w, *ln_out_b; /* [c]            layer_norm_out  */
  const void *z_w, *z_b;         /* [c_z][c], [c_z]  linear_z        */
} gtk_tri_mul_weights;

size_t gtk_tri_mul_packed_size(int64_t c_z, int64_t c, int dtype);
int gtk_tri_mul_pack(const gtk_tri_mul_weights* w, int64_t c_z, int64_t c, int dtype, void* packed,
                     size_t packed_bytes, void* stream);
size_t gtk_tri_mul_workspace_size(int64_t B, int64_t N, int64_t c_z, int64_t c, int dtype);
/* mask may be NULL (all ones).  out may not alias z. */
int gtk_tri_mul_forward(const void* z, const float* mask, void* out, const void* packed, int64_t B,
                        int64_t N, int64_t c_z, int64_t c, int outgoing, int residual,
                        float eps_in, float eps_out, int dtype, void* workspace,
                        size_t workspace_bytes, void* stream);

/* Memory-bounded form of gtk_tri_mul_forward: output rows i run chunk_rows at
 * a time (rounded up to the contraction tile: 64, 128 or 256 rows), the
 * row-chunking of chunk_layer src/genie_tk/utils.py:78-123 applied to the
 * update's output row axis.  The workspace drops from 3 * B*c*Np^2 elements
 * (Np = N rounded up to 64) to B*c*Np^2 + 2 * B*c*R*Np for R chunk rows: the
 * b projections of every row stay resident, the a projections and the
 * contraction of one chunk at a time.  Output bit-identical to
 * gtk_tri_mul_forward.  chunk_rows = 0 (or >= N) runs unchunked.  Every
 * shape and dtype of gtk_tri_mul_forward. */
size_t gtk_tri_mul_workspace_size_chunked(int64_t B, int64_t N, int64_t c_z, int64_t c, int dtype,
                                          int64_t chunk_rows);
int gtk_tri_mul_forward_chunked(const void* z, const float* mask, void* out, const void* packed,
                                int64_t B, int64_t N, int64_t c_z, int64_t c, int outgoing,
                                int residual, float eps_in, float eps_out, int dtype,
                                int64_t chunk_rows, void* workspace, size_t workspace_bytes,
                                void* stream);

/* Experiment (fp8 a/b storage, outside the bf16 parity contract): the
 * forward of gtk_tri_mul_forward with the gated projections a and b stored
 * as OCP fp8 E4M3 (1 byte per element instead of 2, no scaling; values
 * clamped to +-448) and contracted on the fp8 matrix cores
 * (v_mfma_f32_32x32x64_f8f6f4, fp32 accumulation); x and the epilogue stay
 * bf16.  Its error against the fp32 reference is that of 3-bit mantissas in
 * a and b, well beyond the bf16 tolerance; it is reported beside the bf16
 * path, not as it.  bf16 z, c_z = 128, c in {64, 128}; planes padded to N
 * rounded up to 256.  packed: gtk_tri_mul_pack with GTK_BF16.  No
 * counterpart in the reference (whose large-N path is chunk_layer,
 * src/genie_tk/utils.py:78-123). */
size_t gtk_tri_mul_fp8ab_workspace_size(int64_t B, int64_t N, int64_t c_z, int64_t c);
int gtk_tri_mul_forward_fp8ab(const void* z, const float* mask, void* out, const void* packed,
                              int64_t B, int64_t N, int64_t c_z, int64_t c, int outgoing,
                              int residual, float eps_in, float eps_out, void* workspace,
                              size_t workspace_bytes, void* stream);
/* Its contraction alone: x[p][i][j] = sum_k a[p][i][k] * b[p][j][k] over
 * nplanes planes of Np x Np fp8 E4M3 bytes, x in bf16.  Np % 256 == 0. */
int gtk_tri_mul_contract_fp8(const void* a, const void* b, void* x, int64_t nplanes, int64_t Np,
                             void* stream);

/* Backward of gtk_tri_mul_forward (update only, no residual): given dL/dy,
 * writes dL/dz (element type dtype) and the gradient of every parameter
 * (fp32, the nn.Linear / LayerNorm layouts of gtk_tri_mul_weights).  The
 * reference has no backward kernel: its gradients are torch autograd over
 * TriangleMultiplicativeUpdate._forward_pytorch src/genie_tk/triangle_mul.py:103-132,
 * which this computes (forward activations recomputed from z and the raw
 * weights in w).  Gradients are written, not accumulated.  c_z and c each
 * in {32, 64, 128}. */
typedef struct gtk_tri_mul_grads {
  float *ln_in_w, *ln_in_b, *a_p_w, *a_p_b, *a_g_w, *a_g_b, *b_p_w, *b_p_b;
  float *b_g_w, *b_g_b, *g_w, *g_b, *ln_out_w, *ln_out_b, *z_w, *z_b;
} gtk_tri_mul_grads;

size_t gtk_tri_mul_backward_workspace_size(int64_t B, int64_t N, int64_t c_z, int64_t c,
                                           int dtype);
int gtk_tri_mul_backward(const void* z, const float* mask, const void* dy,
                         const gtk_tri_mul_weights* w, void* dz, const gtk_tri_mul_grads* grads,
                         int64_t B, int64_t N, int64_t c_z, int64_t c, int outgoing, float eps_in,
                         float eps_out, int dtype, void* workspace, size_t workspace_bytes,
                         void* stream);

/* ------------------------------------------------------------------------
 * Fused TriangleAttention forward (starting / ending node).
 * Replaces TriangleAttention._forward_cuda src/genie_tk/triangle_attention.py:145-179
 * (semantics of _forward_pytorch :100-143 and Attention.forward
 * src/genie_tk/primitives.py:114-178); ending(x, m) = starting(x^T, m^T)^T.
 *   xn   = LN(x);  tri[h,q,k] = xn[q,k] . W_tri[h]
 *   o    = softmax(q k^T / sqrt(d) + mask_bias + tri) v        per row, head
 *   out  = (o * sigmoid(xn W_g^T + b_g)) W_o^T + b_o    [+ x if residual]
 * mask_bias[k] = inf * (mask[k] - 1) in fp32, the module's constructor
 * argument inf (triangle_attention.py:57,118; the reference default is 1e9):
 * keys with mask == 1 take no bias, any other mask value (0 or fractional)
 * takes that bias, and a row whose keys all carry a bias follows the fp32
 * arithmetic of the reference (uniform attention for inf = 1e9 and mask 0).
 * |inf| <= 1e37.  c_in in {32, 64, 128}, H in {1, 2, 4}, head dim c_h / H in
 * [1, 32] (the reference layer's default c_h = 32, H = 4 is d = 8), N <= 8192.
 * ------------------------------------------------------------------------ */
typedef struct gtk_tri_attn_weights {
  int dtype;                 /* element type of every pointer below */
  const void *ln_w, *ln_b;   /* [c_in]                layer_norm        */
  const void* tri_w;         /* [H][c_in]             linear (no bias)  */
  const void *q_w, *k_w, *v_w; /* [c_h][c_in]         mha.linear_q/k/v  */
  const void *g_w, *g_b;     /* [c_h][c_in], [c_h]    mha.linear_g      */
  const void *o_w, *o_b;     /* [c_in][c_h], [c_in]   mha.linear_o      */
} gtk_tri_attn_weights;

size_t gtk_tri_attn_packed_size(int64_t c_in, int64_t c_h, int64_t H, int dtype);
int gtk_tri_attn_pack(const gtk_tri_attn_weights* w, int64_t c_in, int64_t c_h, int64_t H,
                      int dtype, void* packed, size_t packed_bytes, void* stream);
size_t gtk_tri_attn_workspace_size(int64_t B, int64_t N, int64_t c_in, int64_t c_h, int64_t H,
                                   int dtype);
/* mask may be NULL (all ones).  out may not alias x. */
int gtk_tri_attn_forward(const void* x, const float* mask, void* out, const void* packed,
                         int64_t B, int64_t N, int64_t c_in, int64_t c_h, int64_t H, int starting,
                         int residual, float eps, float inf, int dtype, void* workspace,
                         size_t workspace_bytes, void* stream);

/* Memory-bounded form of gtk_tri_attn_forward: the attention rows are
 * processed chunk_rows at a time, so the q/k/v/gate workspace holds
 * chunk_rows rows instead of N (the N x N x H triangle bias stays whole: it
 * is shared by every row).  The result equals gtk_tri_attn_forward's.  It is
 * the kernel form of the reference's chunk_layer over the row axis
 * (src/genie_tk/utils.py:78-123), which its attention module imports
 * (triangle_attention.py:23) but never calls; there is no reference kernel.
 * chunk_rows = 0, or >= N, is the unchunked operator.  The workspace size
 * query takes the same chunk_rows.  Every shape and dtype of
 * gtk_tri_attn_forward. */
size_t gtk_tri_attn_workspace_size_chunked(int64_t B, int64_t N, int64_t c_in, int64_t c_h,
                                           int64_t H, int64_t chunk_rows, int dtype);
int gtk_tri_attn_forward_chunked(const void* x, const float* mask, void* out, const void* packed,
                                 int64_t B, int64_t N, int64_t c_in, int64_t c_h, int64_t H,
                                 int starting, int residual, float eps, float inf,
                                 int64_t chunk_rows, int dtype, void* workspace,
                                 size_t workspace_bytes, void* stream);

/* Backward of gtk_tri_attn_forward (update only, no residual): given dL/dy,
 * writes dL/dx (element type dtype) and the gradient of every parameter
 * (fp32, the layouts of gtk_tri_attn_weights).  The reference has no backward
 * kernel: its gradients are torch autograd over TriangleAttention._forward_pytorch
 * src/genie_tk/triangle_attention.py:100-143 and Attention.forward
 * src/genie_tk/primitives.py:114-178, which this computes, including autograd's
 * treatment of rows whose keys are all masked (their uniform softmax still
 * passes its gradient to q, k and the triangle bias).  Activations are
 * recomputed from x and the raw weights in w.  Gradients are written, not
 * accumulated.  The mask bias is the reference default's, inf = 1e9, and
 * the mask must be binary: a key with mask == 1 is valid, a key with
 * mask == 0 is masked, and a row with no valid key is uniform.  Other mask
 * values (fractional, or above 1) are not differentiated correctly: the
 * forward gives them the bias inf * (mask - 1), which this backward does
 * not model, so callers must send such masks elsewhere (the genie_tk
 * modules use autograd of their PyTorch path for them).  c_in in
 * {32, 64, 128}, H == 4, d == 32 (c_h == 128), N <= 4096.  Other head
 * shapes (the reference layer's default of four heads of 8, two heads of 8)
 * are computed here by padding: zero q/k/v/gate/output weight columns up
 * to four heads of 32, W_q scaled by sqrt(32 / d) so the scores keep
 * their 1/sqrt(d), the triangle bias of the missing heads zero, and the
 * padded gradients dropped (genie_tk.triangle_attention does this). */
typedef struct gtk_tri_attn_grads {
  float *ln_w, *ln_b, *tri_w, *q_w, *k_w, *v_w, *g_w, *g_b, *o_w, *o_b;
} gtk_tri_attn_grads;

size_t gtk_tri_attn_backward_workspace_size(int64_t B, int64_t N, int64_t c_in, int64_t c_h,
                                            int64_t H, int dtype);
int gtk_tri_attn_backward(const void* x, const float* mask, const void* dy,
                          const gtk_tri_attn_weights* w, void* dx, const gtk_tri_attn_grads* grads,
                          int64_t B, int64_t N, int64_t c_in, int64_t c_h, int64_t H, int starting,
                          float eps, int dtype, void* workspace, size_t workspace_bytes,
                          void* stream);

/* ------------------------------------------------------------------------
 * PairTransition fused with the pair-stack residual and mask.
 * Replaces PairTransition.forward src/genie_tk/pair_transform.py:64-84 and the
 * update of PairTransformLayer.forward :180-193 (p = p + transition(p);
 * p = p * mask):
 *   out = (residual ? p : 0) + (relu(LN(p) W1^T + b1) W2^T + b2),  times mask
 * p, out: [rows][c] (dtype: GTK_BF16 or GTK_F32); mask: [rows] float or
 * NULL.  W1 [n c][c], W2 [c][n c] (nn.Linear layout).  c in {64, 128},
 * n == 4.  The packed weights are built for one dtype (pack and forward
 * with the same dtype).
 * ------------------------------------------------------------------------ */
typedef struct gtk_pair_transition_weights {
  int dtype;                 /* element type of every pointer below */
  const void *ln_w, *ln_b;   /* [c]                   layer_norm         */
  const void *w1, *b1;       /* [n c][c], [n c]       linear_1           */
  const void *w2, *b2;       /* [c][n c], [c]         linear_2           */
} gtk_pair_transition_weights;

size_t gtk_pair_transition_packed_size(int64_t c, int64_t n, int dtype);
int gtk_pair_transition_pack(const gtk_pair_transition_weights* w, int64_t c, int64_t n, int dtype,
                             void* packed, size_t packed_bytes, void* stream);
/* out may not alias p. */
int gtk_pair_transition_forward(const void* p, const float* mask, void* out, const void* packed,
                                int64_t rows, int64_t c, int64_t n, int residual, float eps,
                                int dtype, void* stream);

/* Backward of PairTransition.forward (no residual, no mask): given dL/dy,
 * writes dL/dp (element type dtype) and the gradient of every parameter
 * (fp32, nn.Linear / LayerNorm layouts).  The reference has no backward
 * kernel: its gradients are torch autograd over PairTransition.forward
 * src/genie_tk/pair_transform.py:79-84, which this computes (h recomputed
 * from p; the ReLU passes the gradient where its input is > 0).  w holds the
 * raw parameters (packed into the workspace on each call).  Gradients are
 * written, not accumulated; a NULL gradient pointer skips that output.
 * rows <= 2^31. */
typedef struct gtk_pair_transition_grads {
  float *ln_w, *ln_b, *w1, *b1, *w2, *b2;
} gtk_pair_transition_grads;

size_t gtk_pair_transition_backward_workspace_size(int64_t rows, int64_t c, int64_t n, int dtype);
int gtk_pair_transition_backward(const void* p, const void* dy, const gtk_pair_transition_weights* w,
                                 void* dp, const gtk_pair_transition_grads* g, int64_t rows,
                                 int64_t c, int64_t n, float eps, int dtype, void* workspace,
                                 size_t workspace_bytes, void* stream);

/* ------------------------------------------------------------------------
 * Per-kernel timing (instrumentation; no counterpart in the reference).
 * gtk_timing_enable(1) makes every subsequent launch record a HIP event
 * before and after each kernel on its stream; gtk_timing_report() waits for
 * them and writes one line per kernel name, "name count total_ms min_ms
 * max_ms\n", then clears the records.  gtk_timing_enable(0) stops recording.
 * ------------------------------------------------------------------------ */
int gtk_timing_enable(int on);
int gtk_timing_report(char* buf, size_t buf_bytes);

#ifdef __cplusplus
}
#endif
#endif /* GENIE_TK_H_ */
