/*
 * mlk_hip.h -- C ABI of the MI355X (gfx950) RDT4quant fused-forward kernels.
 *
 * This library replaces, for device-resident tensors, the CPU operators that
 * the reference exposes through its PyTorch extension module montlok._C
 * (rdt4quant_cpu/montlok.cpp, op table at montlok.cpp:1457-1499). Each entry
 * point below names the reference operator it stands in for (file:line).
 *
 * Conventions
 *   - Plain device pointers, element counts and element strides; no torch
 *     types. fp32 tensors unless stated; the last dimension of every tensor
 *     is dense, leading dimensions may be strided where a stride is given.
 *   - Outputs are written into caller-provided device buffers (the Python
 *     layer allocates them with the caching allocator, as montlok.cpp
 *     allocates with torch::empty). No entry point allocates device memory.
 *   - Work is enqueued on `stream` (a hipStream_t) and is stream-ordered; no
 *     entry point synchronises the device.
 *   - Every entry point returns an mlk_status; on failure mlk_last_error()
 *     returns a thread-local message (the reference raises RuntimeError with
 *     the TORCH_CHECK text; the Python layer raises the same text). This
 *     mirrors montlok_status + montlok_last_error of the reference's product
 *     C ABI (include/montlok/montlok.h:16-17,43-52).
 *   - Scalar parameters that the reference reads from 0-d tensors (the mHC
 *     alphas) are passed as device pointers so no call reads device memory
 *     from the host.
 */
#ifndef MLK_HIP_H
#define MLK_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct ihipStream_t* mlk_stream_t; /* identical to hipStream_t */

/* Element type of a weight operand. */
typedef enum mlk_dtype {
    MLK_DTYPE_F32 = 0,
    MLK_DTYPE_BF16 = 1
} mlk_dtype;

/* Attention mask (which keys j a query i sees; queries sit at the trailing
 * q_length of kv_length positions). */
typedef enum mlk_mask {
    MLK_MASK_NONE = 0,                /* every key */
    MLK_MASK_CAUSAL_TOP_LEFT = 1,     /* j <= i (SDPA is_causal) */
    MLK_MASK_CAUSAL_BOTTOM_RIGHT = 2  /* j <= kv_length - q_length + i */
} mlk_mask;

typedef enum mlk_status {
    MLK_OK = 0,
    MLK_ERR_INVALID_ARGUMENT = 1,
    MLK_ERR_RUNTIME = 2,
    MLK_ERR_UNSUPPORTED = 3
} mlk_status;

/* Thread-local message of the last failed call on this thread ("" if none). */
const char* mlk_last_error(void);

/* ABI version of this header (bumped on any signature change). */
int mlk_abi_version(void);

/* JSON object describing the build and the current device: gfx arch, CU
 * count, kernel variant. Replaces build_info() (montlok.cpp:1417-1455).
 * Writes at most `capacity` bytes including the terminating NUL. */
mlk_status mlk_build_info(char* buffer, size_t capacity);

/* Launches a kernel that does nothing, with `blocks` x `threads` and the
 * given dynamic LDS: a diagnostic with no counterpart in the reference. HIP
 * graph nodes of it, in a kernel's launch shape, time the floor that launch
 * pays before any of its work (the measurement reports it beside the step). */
mlk_status mlk_empty_kernel(int64_t blocks, int64_t threads, size_t dynamic_lds_bytes, mlk_stream_t stream);

/* ---------------------------------------------------------------- norms -- */

/* rms_norm(x, weight, eps, groups) -- montlok.cpp:915-938, kernel
 * montlok_layers.h:20-65. x: rows of `dim` floats, `row_stride` apart;
 * out: [rows, dim] contiguous. eps is the Python float (cast through float32
 * as the reference does). groups must divide dim. */
mlk_status mlk_rms_norm(const float* x, int64_t rows, int64_t dim, int64_t row_stride, const float* weight,
                        double eps, int64_t groups, float* out, mlk_stream_t stream);

/* add_rms_norm(left, right, weight, eps, groups) -- montlok.cpp:978-1007,
 * kernel montlok_layers.h:71-90. left/right/residual/normalized: [rows, dim]
 * contiguous. */
mlk_status mlk_add_rms_norm(const float* left, const float* right, int64_t rows, int64_t dim, const float* weight,
                            double eps, int64_t groups, float* residual, float* normalized, mlk_stream_t stream);

/* layer_norm(x, weight, bias, eps) -- montlok.cpp:1057-1082, kernel
 * montlok_layers.h:117-184. bias may be NULL. */
mlk_status mlk_layer_norm(const float* x, int64_t rows, int64_t dim, int64_t row_stride, const float* weight,
                          const float* bias, double eps, float* out, mlk_stream_t stream);

/* layer_norm as mlk_layer_norm computes it (montlok.cpp:1057-1082), each
 * float result then rounded to bf16 (nearest even) into out [rows, dim]: the
 * kv_norm of mla_forward (montlok.cpp:1200) in the form the matrix cores take
 * for its kv_up (:1201), as mlk_mla_attend_normed reads it. Built for 16-byte
 * aligned rows of 4 * 2^k floats (k <= 6); MLK_ERR_UNSUPPORTED otherwise. */
mlk_status mlk_layer_norm_bf16(const float* x, int64_t rows, int64_t dim, int64_t row_stride, const float* weight,
                               const float* bias, double eps, void* out, mlk_stream_t stream);

/* swiglu(x) -- montlok.cpp:942-963, kernel montlok_layers.h:95-112. x rows
 * hold [gate | up] (2*hidden floats, row_stride apart); out: [rows, hidden]. */
mlk_status mlk_swiglu(const float* x, int64_t rows, int64_t hidden, int64_t row_stride, float* out,
                      mlk_stream_t stream);

/* -------------------------------------------------------------- linear -- */

/* linear(input, weight, bias=None) -- linear_dispatch, montlok.cpp:67-91
 * (op table :1458). y[rows, N] = x[rows, K] W[N, K]^T + bias[N].
 * x: fp32 rows `x_stride` floats apart; W: contiguous, fp32 or bf16
 * (weight_dtype, an mlk_dtype); bias: fp32 [N] or NULL; out: fp32 rows
 * `out_stride` floats apart. bf16 weights run on bf16 matrix cores with x
 * rounded to bf16 and fp32 accumulation; fp32 weights stay fp32 throughout. */
mlk_status mlk_linear(const float* x, int64_t rows, int64_t in_features, int64_t x_stride, const void* weight,
                      int32_t weight_dtype, const float* bias, int64_t out_features, float* out,
                      int64_t out_stride, mlk_stream_t stream);

/* linear followed by a residual add: out = residual + (x W^T + bias), the
 * add a separate fp32 rounding, so the result is bit-identical to mlk_linear
 * into a buffer and then residual + that buffer (the x = x + f(norm(x))
 * steps of python/montlok/rdt/reference/Model/blocks.py:66-75). residual:
 * fp32 rows `res_stride` floats apart. No single counterpart in the
 * reference's op table: it fuses linear (montlok.cpp:1458) with the caller's
 * residual add. */
mlk_status mlk_linear_residual(const float* x, int64_t rows, int64_t in_features, int64_t x_stride,
                               const void* weight, int32_t weight_dtype, const float* bias, int64_t out_features,
                               const float* residual, int64_t res_stride, float* out, int64_t out_stride,
                               mlk_stream_t stream);

/* rms_norm(x, norm_weight, eps, groups) then linear(., weight, bias) in one
 * launch, without the normalised intermediate: bit-identical to mlk_rms_norm
 * into a buffer followed by mlk_linear on it. Built for groups of 8, 16, 32
 * or 64 floats and 16-byte aligned x rows, norm weight and weight rows, on
 * the shapes that take the one-wave-per-tile linear (fewer 128-row blocks x
 * 64-column chunks than CUs, in_features <= 256 and a multiple of 8) and, for
 * fp32 weights with in_features 128, on any row count (the row-layout linear
 * with the norm applied to its loaded fragments); other shapes return
 * MLK_ERR_UNSUPPORTED and the caller runs the two operators.
 * No single counterpart in the reference's op table: it fuses rms_norm
 * (montlok.cpp:1481) with the in_proj linear that follows it (stage1_forward,
 * montlok.cpp:1030-1034). */
mlk_status mlk_rms_norm_linear(const float* x, int64_t rows, int64_t in_features, int64_t x_stride,
                               const float* norm_weight, double eps, int64_t groups, const void* weight,
                               int32_t weight_dtype, const float* bias, int64_t out_features, float* out,
                               int64_t out_stride, mlk_stream_t stream);

/* ----------------------------------------------------------------- MLA -- */

/* mla_rope_qk(q, kv, k_rope, cos, sin, nope_dim) -- montlok.cpp:1093-1154,
 * kernel montlok_layers.h:190-234. q: [B, q_length, H, head_dim] tokens
 * `q_token_stride` floats apart, rotated IN PLACE on the last rope_dim =
 * head_dim - nope_dim lanes of every head (rotate_half convention, fp64
 * arithmetic, one rounding); the rows hold the trailing q_length positions.
 * kv: [B, L, H, nope_dim + head_dim] contiguous; k_rope: [B, L, rope_dim]
 * tokens `k_rope_token_stride` apart; cos/sin: [L, rope_dim] contiguous.
 * k: [B, L, H, head_dim] = cat(kv[..., :nope_dim], rope(k_rope)). */
mlk_status mlk_mla_rope_qk(float* q, int64_t q_token_stride, int64_t q_length, const float* kv,
                           const float* k_rope, int64_t k_rope_token_stride, const float* cosine,
                           const float* sine, int64_t batch, int64_t length, int64_t heads, int64_t head_dim,
                           int64_t nope_dim, float* k, mlk_stream_t stream);

/* Scaled dot-product attention, softmax(q k^T * scale) v, per window and
 * head -- the at::scaled_dot_product_attention call of mla_forward
 * (montlok.cpp:1205-1208) and of MLACPU._attend (python/montlok/rdt/mla.py
 * :191-213). q: [B, q_length, H, head_dim], k/v: [B, kv_length, H,
 * head_dim], each with its own token and head strides (dense head_dim);
 * out: [B, q_length, H, head_dim] contiguous. mask: an mlk_mask. precision:
 * MLK_DTYPE_BF16 (bf16 matrix cores, fp32 softmax and accumulation) or
 * MLK_DTYPE_F32 (fp32 throughout). head_dim <= 128. */
mlk_status mlk_attention(const float* q, int64_t q_token_stride, int64_t q_head_stride, const float* k,
                         int64_t k_token_stride, int64_t k_head_stride, const float* v, int64_t v_token_stride,
                         int64_t v_head_stride, int64_t batch, int64_t heads, int64_t q_length, int64_t kv_length,
                         int64_t head_dim, int32_t mask, double scale, int32_t precision, float* out,
                         mlk_stream_t stream);

/* The part of mla_forward between its two projections (montlok.cpp:1196-1209)
 * for the full causal sequence, fused per (window, head): LayerNorm of the
 * latent rows, this head's kv_up slice (bf16 weights), k = cat(k_nope,
 * rope(k_rope)), q's rope lanes rotated, top-left causal attention.
 * projected: in_proj output [B, L, W] with q at column q_offset + h*head_dim,
 * the latent at kv_offset and k_rope at k_rope_offset; kv_up_weight: bf16
 * [H*(nope+hd), kv_rank]; cos/sin: [L, rope]; out: [B, L, H, head_dim]. The
 * result equals mla_rope_qk + mlk_attention (bf16) on the separately
 * computed kv, bit for bit. Built for head_dim 32 / nope 16 (L <= 128) and
 * head_dim 64 / nope 32 (L <= 256), kv_rank 64; MLK_ERR_UNSUPPORTED
 * otherwise. No reference operator of its own. */
mlk_status mlk_mla_attend(const float* projected, int64_t batch, int64_t length, int64_t proj_token_stride,
                          int64_t q_offset, int64_t kv_offset, int64_t k_rope_offset, int64_t heads,
                          int64_t head_dim, int64_t nope_dim, int64_t kv_rank, const float* kv_norm_w,
                          const float* kv_norm_b, double kv_norm_eps, const void* kv_up_weight, const float* cosine,
                          const float* sine, double scale, float* out, mlk_stream_t stream);


/* mlk_mla_attend with the latent already normalised (the part of mla_forward
 * after its kv_norm, montlok.cpp:1201-1209): latent_normed holds bf16 rows
 * [B * L, kv_rank] (mlk_layer_norm_bf16 of the latent columns) and the block
 * skips its LayerNorm, which otherwise every head's block repeats; everything
 * else as mlk_mla_attend, and the same result bit for bit. */
mlk_status mlk_mla_attend_normed(const float* projected, int64_t batch, int64_t length, int64_t proj_token_stride,
                                 int64_t q_offset, int64_t k_rope_offset, int64_t heads, int64_t head_dim,
                                 int64_t nope_dim, int64_t kv_rank, const void* latent_normed,
                                 const void* kv_up_weight, const float* cosine, const float* sine, double scale,
                                 float* out, mlk_stream_t stream);

/* mla_forward(x, in_proj_weight, q_weight, kv_norm_weight, kv_norm_bias,
 * kv_norm_eps, kv_up_weight, out_weight, cos, sin, n_heads, head_dim,
 * nope_dim, kv_lora_rank, n_last = L, causal = true, scale) --
 * montlok.cpp:1159-1211, every causal query: in_proj, kv_norm, kv_up, RoPE,
 * top-left causal attention and the output projection in one launch (one
 * block per window; for 4 heads of 64 one block per window and 64 query
 * rows, walking the key rows up to them), so neither the projection nor the
 * attention output goes through HBM. x: rows of d_model floats, x_token_stride apart within a
 * window and x_batch_stride apart between windows; in_proj_weight [d_model +
 * kv_rank + rope, d_model], kv_up_weight [heads (nope + head_dim), kv_rank]
 * and out_weight [d_model, d_model], all bf16 (weight_dtype MLK_DTYPE_BF16);
 * cos/sin [L, rope]; out [B, L, d_model] contiguous. The result equals the
 * separate path (linear, mlk_layer_norm_bf16, mlk_mla_attend_normed, linear)
 * bit for bit. Built for 8 heads of 32 (nope 16, rope 16), kv_rank 64,
 * L <= 128, and for 4 heads of 64 (nope 32, rope 32), kv_rank 64, L <= 256,
 * with a positive scale and 16-byte aligned operands; MLK_ERR_UNSUPPORTED
 * otherwise. */
mlk_status mlk_mla_forward(const float* x, int64_t batch, int64_t length, int64_t d_model, int64_t x_batch_stride,
                           int64_t x_token_stride, const void* in_proj_weight, const float* kv_norm_w,
                           const float* kv_norm_b, double kv_norm_eps, const void* kv_up_weight,
                           const void* out_weight, const float* cosine, const float* sine, int64_t heads,
                           int64_t head_dim, int64_t nope_dim, int64_t kv_rank, int32_t weight_dtype, double scale,
                           float* out, mlk_stream_t stream);

/* The three bf16 weights of mlk_mla_forward re-laid in its kernel's fragment
 * order, for mlk_mla_forward_packed (no counterpart in the reference: a copy a
 * caller makes once per weight update and keeps). In the row-major layout each
 * fragment load of the kernel reads 16 rows' 64-byte pieces; every block reads
 * all three weights, and those loads bounded the kernel's start and its last
 * head round. mlk_mla_packed_elems: bf16 elements of the packed copy for the
 * geometry (each of the two one-launch geometries has its own layout), 0 where
 * no one-launch kernel is built for it.
 * mlk_mla_pack_weights writes it (16-byte aligned buffers; MLK_ERR_UNSUPPORTED
 * for other geometries or dtypes). mlk_mla_forward_packed is mlk_mla_forward
 * with the packed copy in place of the three weights: same conditions, the
 * same result bit for bit. */
int64_t mlk_mla_packed_elems(int64_t d_model, int64_t heads, int64_t head_dim, int64_t nope_dim, int64_t kv_rank);
mlk_status mlk_mla_pack_weights(const void* in_proj_weight, const void* kv_up_weight, const void* out_weight,
                                int64_t d_model, int64_t heads, int64_t head_dim, int64_t nope_dim, int64_t kv_rank,
                                int32_t weight_dtype, void* packed, mlk_stream_t stream);
mlk_status mlk_mla_forward_packed(const float* x, int64_t batch, int64_t length, int64_t d_model,
                                  int64_t x_batch_stride, int64_t x_token_stride, const void* packed_weights,
                                  const float* kv_norm_w, const float* kv_norm_b, double kv_norm_eps,
                                  const float* cosine, const float* sine, int64_t heads, int64_t head_dim,
                                  int64_t nope_dim, int64_t kv_rank, double scale, float* out, mlk_stream_t stream);

/* ----------------------------------------------------------------- mHC -- */

/* mhc_prepare(streams, norm_w, eps, proj_w, pre_bias, post_bias, res_bias,
 *             pre_alpha, post_alpha, res_alpha, iters, n_streams,
 *             agg_norm_w, agg_norm_eps) -- montlok.cpp:659-691, kernel
 * montlok_mhc.h:198-322.
 *   streams: `tokens` tokens `token_stride` floats apart, each holding n rows
 *            of d floats `stream_stride` apart (0 = the broadcast backbone).
 *   proj_w:  float64 [2n + n*n, d] = cat(pre, post, res projection weights).
 *   alphas:  device pointers to the three fp32 scalars.
 *   agg_norm_w: optional [d] (NULL = no in-place RMSNorm of agg).
 *   outputs: agg [tokens, d], pre [tokens, n], post [tokens, n],
 *            res [tokens, n, n], all contiguous. */
mlk_status mlk_mhc_prepare(const float* streams, int64_t tokens, int64_t n, int64_t d, int64_t stream_stride,
                           int64_t token_stride, const float* norm_w, double eps, const double* proj_w,
                           const float* pre_bias, const float* post_bias, const float* res_bias,
                           const float* pre_alpha, const float* post_alpha, const float* res_alpha,
                           int64_t sinkhorn_iters, const float* agg_norm_w, double agg_norm_eps, float* agg,
                           float* pre, float* post, float* res, mlk_stream_t stream);

/* mhc_combine(streams, res, post, out) -- montlok.cpp:726-739, and
 * mhc_combine_collapse -- montlok.cpp:743-758 (kernel montlok_mhc.h:336-438).
 * new_streams: [tokens, n, d] contiguous or NULL; collapsed: [tokens, d] or
 * NULL (mean over the rounded new streams). At least one must be given.
 * new_streams may be `streams` itself (in place, as montlok_mhc.h:440-497
 * does) when the streams are contiguous [tokens, n, d] and n <= 8; any other
 * overlap between them is not supported. */
mlk_status mlk_mhc_combine(const float* streams, int64_t tokens, int64_t n, int64_t d, int64_t stream_stride,
                           int64_t token_stride, const float* res, const float* post, const float* out,
                           float* new_streams, float* collapsed, mlk_stream_t stream);

/* mhc_combine_prepare(streams, res, post, out, <next hc args>) --
 * montlok.cpp:763-802, kernel montlok_mhc.h:511-522. Writes new_streams
 * [tokens, n, d] and the next residual's agg/pre/post/res. The buffers of the
 * reference's stage-2 variants (montlok.cpp:807-912) are allowed: new_streams
 * may be `streams` itself when the streams are contiguous [tokens, n, d] and
 * n <= 8, post_out and res_out may be `post` and `res`, and agg_out may be
 * `out`; the values are those of distinct buffers. */
mlk_status mlk_mhc_combine_prepare(const float* streams, int64_t tokens, int64_t n, int64_t d,
                                   int64_t stream_stride, int64_t token_stride, const float* res, const float* post,
                                   const float* out, const float* norm_w, double eps, const double* proj_w,
                                   const float* pre_bias, const float* post_bias, const float* res_bias,
                                   const float* pre_alpha, const float* post_alpha, const float* res_alpha,
                                   int64_t sinkhorn_iters, const float* agg_norm_w, double agg_norm_eps,
                                   float* new_streams, float* agg_out, float* pre_out, float* post_out,
                                   float* res_out, mlk_stream_t stream);

/* ------------------------------------------------------------- Mamba-3 -- */

/* Bytes of device workspace mamba3_siso_forward needs: q, k [B,L,H,N],
 * (alpha, beta, gamma) [3,B,L,H] and the rotary angle terms [B,L,H,max(R,1)]
 * (the slab of montlok.cpp:396-420). */
size_t mlk_mamba3_workspace_bytes(int64_t batch, int64_t length, int64_t nheads, int64_t d_state,
                                  int64_t num_rope_angles);

/* mamba3_siso_recurrent(q, k, v, gate, adt, dt, trap_logit, skip) --
 * montlok.cpp:245-325, kernel montlok_kernel.h:251-457. q, k: [B,L,H,N];
 * v, gate: [B,L,H,D] (gate = z * sigmoid(z)); adt, dt, trap_logit: [B,L,H];
 * each with element strides {b, t, h} (3 int64 on the host) and a dense last
 * dimension. skip: [H]. out: [B,L,H,D] contiguous. workspace: 3*B*L*H floats. */
mlk_status mlk_mamba3_siso_recurrent(const float* q, const int64_t* q_strides, const float* k,
                                     const int64_t* k_strides, const float* v, const int64_t* v_strides,
                                     const float* gate, const int64_t* gate_strides, const float* adt,
                                     const int64_t* adt_strides, const float* dt, const int64_t* dt_strides,
                                     const float* trap_logit, const int64_t* trap_strides, const float* skip,
                                     int64_t batch, int64_t length, int64_t heads, int64_t d_state,
                                     int64_t headdim, float* out, void* workspace, size_t workspace_bytes,
                                     mlk_stream_t stream);

/* mlk_mamba3_siso_recurrent without a workspace argument, for callers that
 * cannot allocate device memory (code under HIP graph capture, tight serving
 * loops, harnesses that forbid hipMalloc). No counterpart in the reference.
 * Same arguments, checks and result (bit for bit) as
 * mlk_mamba3_siso_recurrent; the (alpha, beta, gamma) coefficients live in a
 * static device array of MLK_NOALLOC_SCRATCH_BYTES that each GPU holds from
 * library load to process end, so batch * length * heads may be at most
 * MLK_NOALLOC_SCRATCH_BYTES / 12 (699,050); larger calls fail with
 * MLK_ERR_INVALID_ARGUMENT. The entry point calls no allocating routine.
 * All calls on one GPU share its array, and the library orders them: each
 * call's stream first waits on an event that the previous call recorded on
 * its own stream after using the array (a mutex orders the enqueues of host
 * threads). Under HIP graph capture no event is waited on or recorded (a
 * capture cannot wait on work outside it): a captured call is ordered only by
 * its graph, so a graph holding it must not be replayed while another call on
 * that GPU may run. The first call on each device (which looks the array's
 * address up and creates its event) must happen outside capture. */
#define MLK_NOALLOC_SCRATCH_BYTES (8u << 20)
mlk_status mlk_mamba3_siso_recurrent_noalloc(const float* q, const int64_t* q_strides, const float* k,
                                             const int64_t* k_strides, const float* v, const int64_t* v_strides,
                                             const float* gate, const int64_t* gate_strides, const float* adt,
                                             const int64_t* adt_strides, const float* dt, const int64_t* dt_strides,
                                             const float* trap_logit, const int64_t* trap_strides, const float* skip,
                                             int64_t batch, int64_t length, int64_t heads, int64_t d_state,
                                             int64_t headdim, float* out, mlk_stream_t stream);

/* mamba3_siso_forward(projected, gate, B_bias, C_bias, B_norm_w, C_norm_w,
 * dt_bias, D, d_state, ngroups, nheads, headdim, num_rope_angles, b_eps,
 * c_eps, a_floor) -- montlok.cpp:333-492, kernels montlok_kernel.h:463-597
 * and :251-457. projected: [B,L,W] in_proj output with batch/token strides
 * (W = 2*d_inner + 2*G*N + 3*H + R, dense last dim); gate: NULL (silu of the
 * z lanes in the kernel, double, rounded once) or [B,L,d_inner] with strides.
 * out: [B,L,d_inner] contiguous. */
mlk_status mlk_mamba3_siso_forward(const float* projected, int64_t batch, int64_t length, int64_t width,
                                   int64_t proj_batch_stride, int64_t proj_token_stride, const float* gate,
                                   int64_t gate_batch_stride, int64_t gate_token_stride, const float* b_bias,
                                   const float* c_bias, const float* b_norm_w, const float* c_norm_w,
                                   const float* dt_bias, const float* skip, int64_t d_state, int64_t ngroups,
                                   int64_t nheads, int64_t headdim, int64_t num_rope_angles, double b_eps,
                                   double c_eps, double a_floor, float* out, void* workspace,
                                   size_t workspace_bytes, mlk_stream_t stream);

/* The mixer of the RMSNorm -> Mamba-3 residual block in one launch:
 *   out = mamba3_siso_forward(in_proj(GroupedRMSNorm(x)))
 * with the in-kernel silu gate: rms_norm (montlok.cpp:915-938), the in_proj
 * linear and mamba3_siso_forward (montlok.cpp:333-492) of the Mamba3Layer
 * forward (reference/Model/layers/mamba3_layer.py:488-498; mamba3_siso_layer,
 * montlok.cpp:496-519, without its out_proj). No single counterpart in the
 * reference's op table. x: [B, L, d_model] with batch/token strides (dense
 * last dim); norm_w [d_model] (norm_groups groups, eps cast through float32);
 * in_weight [W, d_model] fp32 (in_dtype: mlk_dtype); the mixer's parameters
 * and geometry as mlk_mamba3_siso_forward; out: [B, L, d_inner] contiguous.
 * One block per (window, head) computes the in_proj columns its head reads
 * into LDS and runs the chunked scan from there, so the in_proj rows never
 * reach memory. The result equals mlk_rms_norm_linear ->
 * mlk_mamba3_siso_forward bit for bit where mlk_rms_norm_linear takes its
 * one-wave-per-tile form. Built for d_state 16 with heads of 32, d_model <= 64
 * in RMSNorm groups of 8, 3 * nheads + num_rope_angles <= 16, one B/C group,
 * fp32 in_proj weights and 16-byte aligned x rows; MLK_ERR_UNSUPPORTED
 * otherwise (the caller then runs the two operators). The block is this,
 * then mlk_linear_residual for out_proj + x. */
mlk_status mlk_rms_norm_mamba3_forward(const float* x, int64_t batch, int64_t length, int64_t d_model,
                                       int64_t x_batch_stride, int64_t x_token_stride, const float* norm_w,
                                       double norm_eps, int64_t norm_groups, const void* in_weight, int32_t in_dtype,
                                       const float* b_bias, const float* c_bias, const float* b_norm_w,
                                       const float* c_norm_w, const float* dt_bias, const float* skip,
                                       int64_t d_state, int64_t ngroups, int64_t nheads, int64_t headdim,
                                       int64_t num_rope_angles, double b_eps, double c_eps, double a_floor,
                                       float* out, mlk_stream_t stream);

/* One token of the same layer for `streams` independent sequences with
 * carried state. No reference operator exists (the reference kernel keeps the
 * state inside one call, montlok_kernel.h:257-259); this is the state the
 * sequence kernel carries, made explicit, in the shape of the upstream step
 * API (u, angle_state, ssm_state, k_state, v_state) of
 * reference/Model/layers/mamba3_layer.py:567-580. projected: [S, W] rows
 * `proj_stride` apart. State, updated in place: ssm [S,H,N,D], k [S,H,N],
 * v [S,H,D] (fp32), angle [S,H,max(R,1)] (fp64 running phase sum).
 * started = 0 for the first token of a zero state. out: [S, H*D].
 * Stepping T tokens from a zero state reproduces mamba3_siso_forward over the
 * T tokens. headdim <= 64, d_state <= 128. */
mlk_status mlk_mamba3_siso_step(const float* projected, int64_t streams, int64_t proj_stride, const float* b_bias,
                                const float* c_bias, const float* b_norm_w, const float* c_norm_w,
                                const float* dt_bias, const float* skip, int64_t d_state, int64_t ngroups,
                                int64_t nheads, int64_t headdim, int64_t num_rope_angles, double b_eps, double c_eps,
                                double a_floor, float* ssm_state, float* k_state, float* v_state,
                                double* angle_state, int started, float* out, mlk_stream_t stream);

/* --------------------------------------------------------- diagnostics -- */

/* Evaluates the kernels' device math helpers on x[count] (float64):
 * out[0:count] = exp, out[count:2count] = tanh, out[2count:3count] =
 * sigmoid, out[3count:4count] = 1/x (for positive x). No reference operator;
 * it plays the role of the reference self-test of its own polynomial exp
 * (rdt4quant_cpu/montlok_selftest.cpp:770-790). */
mlk_status mlk_math_check(const double* x, int64_t count, double* out, mlk_stream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* MLK_HIP_H */
