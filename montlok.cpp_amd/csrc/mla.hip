// Multi-head latent attention: the rotary key assembly and the attention
// contraction.
//
// mla_rope_qk (rdt4quant_cpu/montlok.cpp:1093-1154, kernel
// montlok_layers.h:190-234): rotate_half RoPE on the last rope_dim lanes of
// every q head (in place) and k = cat(k_nope, rope(k_rope)) per head, fp64
// arithmetic rounded to fp32 once. Query rows may cover only the trailing
// q_length positions; position = token % L.
//
// Attention stands in for the at::scaled_dot_product_attention call of
// mla_forward (montlok.cpp:1205-1208) and F.scaled_dot_product_attention in
// MLACPU._attend (python/montlok/rdt/mla.py:191-213): softmax(q k^T * scale)
// v per (window, head), with the three masks the reference uses (top-left
// causal, none for a single trailing query, bottom-right for several trailing
// queries).
//
// Attention layout. One block = one (window, head, 128 queries); each of its
// four waves owns two 16-query tiles (tile w and 7-w, which balances the
// causal triangle). Keys stream through LDS in chunks of 64 with an online
// softmax. The kernel computes S^T = K Q^T so that the probabilities land in
// the B-operand layout of O^T = V^T P^T: lane l holds query l%16 and keys
// 16t + 4(l/16) + v of every 16-key tile t, and those 8 values (two tiles) are
// exactly the 8 k-slots the next MFMA needs. Only V has to be laid out
// transposed in LDS. Running max, running sum and rescale are per lane. With
// a positive scale s (every MLA caller's), a chunk's max is taken over the raw
// scores and scaled once (RN(max x) s = max RN(x s): rounding is monotone) and
// each exponent is one fma, exp2(x s - m) rounded once; otherwise the scores
// are scaled first and exp2(RN(x s) - m) is formed.
//   BF16: v_mfma_f32_16x16x32_bf16, q/k/v and p rounded to bf16, fp32
//         accumulation and fp32 softmax (bf16-weight configurations).
//   FP32: v_mfma_f32_16x16x4_f32, fp32 throughout (fp32 configurations).

#include <initializer_list>

#include "mlk_common.h"

namespace mlk {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef unsigned short u16;

// ------------------------------------------------------------------ rope

struct RopeArgs {
    float* q;
    int64_t q_ts, q_length;
    const float* kv;
    const float* k_rope;
    int64_t k_rope_ts;
    const float* cosine;
    const float* sine;
    float* k;
    int64_t batch, length, heads, head_dim, nope_dim;
};

// One thread per (token, head, lane j): j < nope copies k_nope; nope <= j <
// nope + rope/2 rotates the pair (i, i + rope/2), i = j - nope, of k and q.
// I: index type of the flat thread index, 32-bit when it fits (cheap divisions).
template <typename I>
__global__ __launch_bounds__(256) void rope_kernel(RopeArgs p) {
    const I per_head = static_cast<I>(p.nope_dim + (p.head_dim - p.nope_dim) / 2);
    const I idx = static_cast<I>(blockIdx.x) * 256 + threadIdx.x;
    if (static_cast<int64_t>(idx) >= p.batch * p.length * p.heads * static_cast<int64_t>(per_head)) return;
    const I th_i = idx / per_head;  // token * heads + h
    const int64_t j = idx - th_i * per_head;
    const I heads = static_cast<I>(p.heads), length = static_cast<I>(p.length);
    const I token_i = th_i / heads;
    const int64_t th = th_i;
    const int64_t h = th_i - token_i * heads;
    const I seq_i = token_i / length;
    const int64_t token = token_i;
    const int64_t pos = token_i - seq_i * length;
    const int64_t seq = seq_i;
    const int64_t rope_dim = p.head_dim - p.nope_dim;
    const int64_t half = rope_dim / 2;
    float* kh = p.k + th * p.head_dim;
    if (j < p.nope_dim) {
        kh[j] = p.kv[th * (p.nope_dim + p.head_dim) + j];
        return;
    }
    const int64_t i = j - p.nope_dim;
    const float* c = p.cosine + pos * rope_dim;
    const float* s = p.sine + pos * rope_dim;
    const float* kr = p.k_rope + token * p.k_rope_ts;
    {
        const double x1 = static_cast<double>(kr[i]);
        const double x2 = static_cast<double>(kr[i + half]);
        kh[p.nope_dim + i] = static_cast<float>(__dsub_rn(__dmul_rn(x1, static_cast<double>(c[i])),
                                                          __dmul_rn(x2, static_cast<double>(s[i]))));
        kh[p.nope_dim + i + half] = static_cast<float>(__dadd_rn(__dmul_rn(x2, static_cast<double>(c[i + half])),
                                                                 __dmul_rn(x1, static_cast<double>(s[i + half]))));
    }
    const int64_t q_first = p.length - p.q_length;
    if (pos >= q_first) {
        float* qh = p.q + (seq * p.q_length + pos - q_first) * p.q_ts + h * p.head_dim + p.nope_dim;
        const double x1 = static_cast<double>(qh[i]);
        const double x2 = static_cast<double>(qh[i + half]);
        const float o1 = static_cast<float>(__dsub_rn(__dmul_rn(x1, static_cast<double>(c[i])),
                                                      __dmul_rn(x2, static_cast<double>(s[i]))));
        const float o2 = static_cast<float>(__dadd_rn(__dmul_rn(x2, static_cast<double>(c[i + half])),
                                                      __dmul_rn(x1, static_cast<double>(s[i + half]))));
        qh[i] = o1;
        qh[i + half] = o2;
    }
}

// ------------------------------------------------------------- attention

struct AttnArgs {
    const float* q;
    int64_t q_ts, q_hs;  // element strides of a query token and of a head within it
    const float* k;
    int64_t k_ts, k_hs;
    const float* v;
    int64_t v_ts, v_hs;
    float* out;  // [B, Lq, H, hd] contiguous
    int64_t batch, heads, q_length, kv_length, head_dim;
    int64_t offset;    // key j is visible to query i iff j <= i + offset
    float scale_log2;  // softmax scale * log2(e)
};

constexpr int kKeysPerChunk = 64;
constexpr int kQueriesPerBlock = 128;

template <bool BF16>
struct AttnElem;
template <>
struct AttnElem<true> {
    using T = u16;
    static constexpr int kPad = 8;
    static __device__ __forceinline__ T from(float x) { return __builtin_bit_cast(u16, static_cast<__bf16>(x)); }
};
template <>
struct AttnElem<false> {
    using T = float;
    static constexpr int kPad = 4;
    static __device__ __forceinline__ T from(float x) { return x; }
};

// 8 consecutive floats of one row (zero where col >= head_dim or !valid).
__device__ __forceinline__ void load_row8(const float* row, int64_t col, int64_t head_dim, bool valid, bool vec,
                                          float (&v)[8]) {
    if (valid && vec && col + 8 <= head_dim) {
        const float4 a = *reinterpret_cast<const float4*>(row + col);
        const float4 b = *reinterpret_cast<const float4*>(row + col + 4);
        v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
        v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
    } else {
#pragma unroll
        for (int j = 0; j < 8; ++j) v[j] = (valid && col + j < head_dim) ? row[col + j] : 0.0f;
    }
}

__device__ __forceinline__ float xor_max(float x, int mask) { return fmaxf(x, __shfl_xor(x, mask)); }
__device__ __forceinline__ float xor_sum(float x, int mask) { return x + __shfl_xor(x, mask); }

// The value of lane l ^ 16 (l ^ 32) through the gfx950 row swaps, VALU
// operations instead of an LDS permute: permlane16_swap(x, x) leaves rows
// {0, 0, 2, 2} in its first result and {1, 1, 3, 3} in its second (a row is 16
// lanes), permlane32_swap(x, x) halves {0, 0} and {1, 1}.
__device__ __forceinline__ float lane_xor16(float x) {
    const int b = __float_as_int(x);
    const auto r = __builtin_amdgcn_permlane16_swap(b, b, false, false);
    return __int_as_float((threadIdx.x & 16) ? r[0] : r[1]);
}
__device__ __forceinline__ float lane_xor32(float x) {
    const int b = __float_as_int(x);
    const auto r = __builtin_amdgcn_permlane32_swap(b, b, false, false);
    return __int_as_float((threadIdx.x & 32) ? r[0] : r[1]);
}

template <int HD, bool BF16, bool VEC, bool RAWMAX>
__global__ __launch_bounds__(256) void attn_kernel(AttnArgs p) {
    using E = AttnElem<BF16>;
    using T = typename E::T;
    constexpr int kPad = E::kPad;
    constexpr int KP = HD + kPad;             // k_lds row pitch (keys x hd)
    constexpr int VP = kKeysPerChunk + kPad;  // vt_lds row pitch (hd x keys)
    constexpr int HC = HD / 32;               // 32-wide hd chunks of S
    constexpr int OT = HD / 16;               // 16-wide hd tiles of O
    __shared__ __attribute__((aligned(16))) T k_lds[kKeysPerChunk * KP];
    __shared__ __attribute__((aligned(16))) T vt_lds[HD * VP];

    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int li = lane & 15;  // query within a tile / row within an operand
    const int g = lane >> 4;   // lane group
    const int64_t h = blockIdx.y;
    const int64_t b = blockIdx.z;
    const int64_t qblock = static_cast<int64_t>(blockIdx.x) * kQueriesPerBlock;
    const int tiles[2] = {wave, 7 - wave};

    // Q as the B operand of S^T = K Q^T: lane holds q[q0 + li][32c + 8g .. +7].
    bf16x8 qb[2][HC];
    float qf[2][BF16 ? 1 : HC][8];
    float m_run[2], l_run[2];
    f32x4 acc[2][OT];
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const int64_t qi = qblock + 16 * tiles[i] + li;
        const bool valid = qi < p.q_length;
        const float* row = p.q + (b * p.q_length + (valid ? qi : 0)) * p.q_ts + h * p.q_hs;
#pragma unroll
        for (int c = 0; c < HC; ++c) {
            float v[8];
            load_row8(row, 32 * c + 8 * g, p.head_dim, valid, VEC, v);
            if constexpr (BF16) {
#pragma unroll
                for (int j = 0; j < 8; ++j) qb[i][c][j] = static_cast<__bf16>(v[j]);
            } else {
#pragma unroll
                for (int j = 0; j < 8; ++j) qf[i][c][j] = v[j];
            }
        }
        m_run[i] = -INFINITY;
        l_run[i] = 0.0f;
#pragma unroll
        for (int t = 0; t < OT; ++t) acc[i][t] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    }

    const int64_t q_last = (qblock + kQueriesPerBlock - 1 < p.q_length ? qblock + kQueriesPerBlock : p.q_length) - 1;
    const int64_t key_end = (q_last + p.offset + 1 < p.kv_length) ? q_last + p.offset + 1 : p.kv_length;

    for (int64_t kbase = 0; kbase < key_end; kbase += kKeysPerChunk) {
        __syncthreads();
        // Stage K (keys x hd) and V^T (hd x keys) of this chunk.
        for (int u = threadIdx.x; u < kKeysPerChunk * (HD / 8); u += 256) {
            const int r = u / (HD / 8);
            const int c8 = (u % (HD / 8)) * 8;
            const int64_t key = kbase + r;
            const bool valid = key < p.kv_length;
            const int64_t tok = b * p.kv_length + (valid ? key : 0);
            float kv8[8];
            load_row8(p.k + tok * p.k_ts + h * p.k_hs, c8, p.head_dim, valid, VEC, kv8);
#pragma unroll
            for (int j = 0; j < 8; ++j) k_lds[r * KP + c8 + j] = E::from(kv8[j]);
            load_row8(p.v + tok * p.v_ts + h * p.v_hs, c8, p.head_dim, valid, VEC, kv8);
#pragma unroll
            for (int j = 0; j < 8; ++j) vt_lds[(c8 + j) * VP + r] = E::from(kv8[j]);
        }
        __syncthreads();

#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const int64_t q0 = qblock + 16 * tiles[i];
            if (q0 >= p.q_length || kbase > q0 + 15 + p.offset) continue;  // tile done or chunk fully masked
            // S^T tiles: s[t][v] = S[query q0 + li][key kbase + 16t + 4g + v].
            f32x4 s[4];
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                s[t] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
                for (int c = 0; c < HC; ++c) {
                    const T* src = k_lds + (16 * t + li) * KP + 32 * c + 8 * g;
                    if constexpr (BF16) {
                        const bf16x8 a = __builtin_bit_cast(bf16x8, *reinterpret_cast<const uint4*>(src));
                        s[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, qb[i][c], s[t], 0, 0, 0);
                    } else {
                        const float4 a0 = *reinterpret_cast<const float4*>(src);
                        const float4 a1 = *reinterpret_cast<const float4*>(src + 4);
                        const float a[8] = {a0.x, a0.y, a0.z, a0.w, a1.x, a1.y, a1.z, a1.w};
#pragma unroll
                        for (int j = 0; j < 8; ++j) {
                            s[t] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[j], qf[i][c][j], s[t], 0, 0, 0);
                        }
                    }
                }
            }
            // Scale, mask, chunk max.
            const int64_t qpos = q0 + li;
            float mx = -INFINITY;
#pragma unroll
            for (int t = 0; t < 4; ++t) {
#pragma unroll
                for (int v = 0; v < 4; ++v) {
                    const int64_t key = kbase + 16 * t + 4 * g + v;
                    const bool ok = key < p.kv_length && key <= qpos + p.offset;
                    const float x = ok ? (RAWMAX ? s[t][v] : s[t][v] * p.scale_log2) : -INFINITY;
                    s[t][v] = x;
                    mx = fmaxf(mx, x);
                }
            }
            mx = xor_max(mx, 16);
            mx = xor_max(mx, 32);
            if constexpr (RAWMAX) mx *= p.scale_log2;  // the max of the scaled scores (the scale is positive)
            const float m_new = fmaxf(m_run[i], mx);
            const float m_use = m_new == -INFINITY ? 0.0f : m_new;
            const float corr = __builtin_amdgcn_exp2f(m_run[i] - m_use);
            m_run[i] = m_new;
            float psum = 0.0f;
#pragma unroll
            for (int t = 0; t < 4; ++t) {
#pragma unroll
                for (int v = 0; v < 4; ++v) {
                    const float e = __builtin_amdgcn_exp2f(RAWMAX ? fmaf(s[t][v], p.scale_log2, -m_use) : s[t][v] - m_use);
                    s[t][v] = e;
                    psum += e;
                }
            }
            l_run[i] = l_run[i] * corr + psum;  // per-lane partial; lane groups summed at the end
#pragma unroll
            for (int t = 0; t < OT; ++t) {
#pragma unroll
                for (int v = 0; v < 4; ++v) acc[i][t][v] *= corr;
            }
            // O^T += V^T P^T over two 32-key halves of the chunk.
#pragma unroll
            for (int half = 0; half < 2; ++half) {
                const f32x4& p0 = s[2 * half];
                const f32x4& p1 = s[2 * half + 1];
#pragma unroll
                for (int t = 0; t < OT; ++t) {
                    const T* vrow = vt_lds + (16 * t + li) * VP + 32 * half + 4 * g;
                    if constexpr (BF16) {
                        bf16x8 pb;
#pragma unroll
                        for (int v = 0; v < 4; ++v) {
                            pb[v] = static_cast<__bf16>(p0[v]);
                            pb[4 + v] = static_cast<__bf16>(p1[v]);
                        }
                        const uint2 lo = *reinterpret_cast<const uint2*>(vrow);
                        const uint2 hi = *reinterpret_cast<const uint2*>(vrow + 16);
                        const uint4 raw = {lo.x, lo.y, hi.x, hi.y};
                        const bf16x8 a = __builtin_bit_cast(bf16x8, raw);
                        acc[i][t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, pb, acc[i][t], 0, 0, 0);
                    } else {
                        const float4 lo = *reinterpret_cast<const float4*>(vrow);
                        const float4 hi = *reinterpret_cast<const float4*>(vrow + 16);
                        const float a[8] = {lo.x, lo.y, lo.z, lo.w, hi.x, hi.y, hi.z, hi.w};
                        const float pv[8] = {p0[0], p0[1], p0[2], p0[3], p1[0], p1[1], p1[2], p1[3]};
#pragma unroll
                        for (int j = 0; j < 8; ++j) {
                            acc[i][t] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[j], pv[j], acc[i][t], 0, 0, 0);
                        }
                    }
                }
            }
        }
    }

    // Normalise and store: acc[i][t][v] = O[query q0 + li][hd 16t + 4g + v].
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const int64_t qi = qblock + 16 * tiles[i] + li;
        float l = xor_sum(l_run[i], 16);
        l = xor_sum(l, 32);
        if (qi >= p.q_length) continue;
        const float inv = 1.0f / l;
        float* orow = p.out + ((b * p.q_length + qi) * p.heads + h) * p.head_dim;
#pragma unroll
        for (int t = 0; t < OT; ++t) {
            const int64_t col = 16 * t + 4 * g;
            const float o[4] = {acc[i][t][0] * inv, acc[i][t][1] * inv, acc[i][t][2] * inv, acc[i][t][3] * inv};
            if (VEC && col + 4 <= p.head_dim) {
                *reinterpret_cast<float4*>(orow + col) = make_float4(o[0], o[1], o[2], o[3]);
            } else {
#pragma unroll
                for (int v = 0; v < 4; ++v) {
                    if (col + v < p.head_dim) orow[col + v] = o[v];
                }
            }
        }
    }
}

template <int HD, bool BF16>
void launch_attn(const AttnArgs& p, bool vec, hipStream_t stream) {
    const dim3 grid(static_cast<unsigned>(ceil_div(p.q_length, kQueriesPerBlock)), static_cast<unsigned>(p.heads),
                    static_cast<unsigned>(p.batch));
    const bool raw = p.scale_log2 > 0.0f;
    if (vec && raw) {
        hipLaunchKernelGGL((attn_kernel<HD, BF16, true, true>), grid, dim3(256), 0, stream, p);
    } else if (vec) {
        hipLaunchKernelGGL((attn_kernel<HD, BF16, true, false>), grid, dim3(256), 0, stream, p);
    } else if (raw) {
        hipLaunchKernelGGL((attn_kernel<HD, BF16, false, true>), grid, dim3(256), 0, stream, p);
    } else {
        hipLaunchKernelGGL((attn_kernel<HD, BF16, false, false>), grid, dim3(256), 0, stream, p);
    }
}

template <bool BF16>
void dispatch_attn(const AttnArgs& p, bool vec, hipStream_t stream) {
    if (p.head_dim <= 32) {
        launch_attn<32, BF16>(p, vec, stream);
    } else if (p.head_dim <= 64) {
        launch_attn<64, BF16>(p, vec, stream);
    } else {
        launch_attn<128, BF16>(p, vec, stream);
    }
}

bool aligned16(const void* ptr) { return (reinterpret_cast<uintptr_t>(ptr) & 15) == 0; }

// ---------------------------------------------------- fused latent attention

// The part of mla_forward between the two projections, for one (window,
// head) per block: LayerNorm of the window's latent rows, this head's slice
// of kv_up on the matrix cores, k = cat(k_nope, rope(k_rope)), q's rope lanes
// rotated, causal attention, all staged in LDS, so neither the normalised
// latent, kv, k nor the rotated q goes through HBM. Every value is computed
// with the operations of the separate kernels (layer_norm_vec_kernel with 16
// lanes per row, linear_kernel's bf16 MFMA over k steps of 32, rope_kernel's
// fp64 rotation, attn_kernel's softmax), so the output is bit-identical to
// the unfused path. Blocks are mapped so that the heads of one window run on
// one XCD and share its L2 copy of the window's latent rows.
struct MlaAttendArgs {
    const float* proj;  // in_proj output rows [B, L, W]
    int64_t proj_ts;    // W
    int64_t q_off, kv_off, kr_off;
    const float* ln_w;
    const float* ln_b;  // may be null
    double ln_eps;
    const u16* w_up;  // [H * (nope + hd), kv_rank] bf16
    const float* cosine;
    const float* sine;
    float* out;  // [B, L, H, hd]
    int64_t batch, heads, length;
    float scale_log2;
    const u16* latent;  // LNIN form: LayerNorm(kv_latent) rows [B * L, kv_rank], bf16
};

// The four-wave form keeps three blocks per CU (its LDS allows three): the
// register budget is held to 168 so that the up-front loads do not cost a
// block.
// LNIN: the latent rows arrive normalised, in bf16 (the in_proj's LayerNorm
// epilogue, the same arithmetic as below), and the block skips its LayerNorm.
template <int HD, int NOPE, int KV, int NW, int TPW, bool LNIN, bool RAWMAX>
__global__ __launch_bounds__(64 * NW) __attribute__((amdgpu_waves_per_eu(NW == 4 ? 3 : 1)))
void mla_attend_kernel(MlaAttendArgs p) {
    constexpr int THREADS = 64 * NW;
    constexpr int ROPE = HD - NOPE, HALF = ROPE / 2;
    constexpr int LMAX = 16 * NW * TPW;  // NW waves x TPW query tiles x 16
    constexpr int UPW = NOPE + HD;       // kv_up rows of one head
    constexpr int XP = KV + 8;           // LDS pitches in bf16 elements (+16 bytes)
    constexpr int KP = HD + 8;
    constexpr int VP = LMAX + 8;
    constexpr int HC = HD / 32;
    constexpr int OT = HD / 16;
    static_assert(HD <= KV && KV == 64 && HD % 32 == 0 && UPW % 16 == 0 && NOPE % 4 == 0 && HALF % 4 == 0,
                  "geometry");
    // LN(kv_latent), then q (pitch KP); the LNIN form keeps only q here (its
    // kv_up operands go from memory into registers).
    __shared__ __attribute__((aligned(16))) u16 xq_s[LMAX * (LNIN ? KP : XP)];
    __shared__ __attribute__((aligned(16))) u16 wu_s[UPW * XP];
    __shared__ __attribute__((aligned(16))) u16 k_s[LMAX * KP];
    __shared__ __attribute__((aligned(16))) u16 vt_s[HD * VP];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int li = lane & 15;
    const int g = lane >> 4;
    const int L = static_cast<int>(p.length);
    const int H = static_cast<int>(p.heads);
    int64_t b, h;
    {
        const int64_t id = blockIdx.x;
        if (p.batch % 8 == 0) {  // XCD x = id % 8 takes windows x, x + 8, ...
            const int64_t k = id / 8;
            b = id % 8 + 8 * (k / H);
            h = k % H;
        } else {
            b = id / H;
            h = id % H;
        }
    }
    const float* rows = p.proj + b * L * p.proj_ts;
    auto rot = [](double x1, double x2, double c1, double s1, double c2, double s2, u16& o1, u16& o2) {
        o1 = AttnElem<true>::from(static_cast<float>(__dsub_rn(__dmul_rn(x1, c1), __dmul_rn(x2, s1))));
        o2 = AttnElem<true>::from(static_cast<float>(__dadd_rn(__dmul_rn(x2, c2), __dmul_rn(x1, s2))));
    };

    // 1. Every global operand of the block is fetched first, with compile-time
    // trip counts and no branch around a load (rows past L read row L - 1, in
    // bounds, and their values are zeroed where they are stored), so the block
    // waits for one round of memory latency rather than one per phase: the
    // latent rows (16 lanes per row, 4 columns each), this head's kv_up rows,
    // k_rope and q of this head, and the cos/sin of their rows, which the k
    // and q rotations share (both map unit u to row u / (HALF / 4) and the
    // pairs from 4 (u % (HALF / 4)) on).
    constexpr int WUN = UPW * (KV / 8);  // 16-byte units of this head's kv_up rows
    constexpr int WUI = (WUN + THREADS - 1) / THREADS;
    constexpr int PASSES = LMAX / (THREADS / 16);
    constexpr int QU = HALF / 4;  // quads of rotary pairs per row
    static_assert((LMAX * QU) % THREADS == 0, "rope units must split evenly");
    constexpr int RI = LMAX * QU / THREADS;
    constexpr int QN = NOPE / 4;
    static_assert((LMAX * QN) % THREADS == 0, "q units must split evenly");
    constexpr int NI = LMAX * QN / THREADS;
    const int lr = tid >> 4, lc = tid & 15;
    // LNIN: wave w computes kv_up for the row tiles w + NW j, and loads their
    // A fragments (row 16 (w + NW j) + l, k = 32 ks + 8 g) of the normalised
    // latent straight into registers.
    constexpr int RPW = LMAX / 16 / NW;
    static_assert(!LNIN || (LMAX / 16) % NW == 0, "kv_up row tiles must split evenly over the waves");
    float4 xs[LNIN ? 1 : PASSES];
    uint4 afr[LNIN ? RPW : 1][KV / 32];
    if constexpr (LNIN) {
#pragma unroll
        for (int j = 0; j < RPW; ++j) {
            const int row = 16 * (wave + NW * j) + li, rc = row < L ? row : L - 1;
#pragma unroll
            for (int ks = 0; ks < KV / 32; ++ks) {
                afr[j][ks] = *reinterpret_cast<const uint4*>(p.latent + (b * L + rc) * static_cast<int64_t>(KV) + 32 * ks + 8 * g);
            }
        }
    } else {
#pragma unroll
        for (int ps = 0; ps < PASSES; ++ps) {
            const int row = ps * (THREADS / 16) + lr;
            const int rc = row < L ? row : L - 1;
            xs[ps] = *reinterpret_cast<const float4*>(rows + rc * p.proj_ts + p.kv_off + 4 * lc);
        }
    }
    uint4 wur[WUI];
#pragma unroll
    for (int it = 0; it < WUI; ++it) {
        const int u = min(tid + it * THREADS, WUN - 1);
        const int r = u / (KV / 8), c = (u % (KV / 8)) * 8;
        wur[it] = *reinterpret_cast<const uint4*>(p.w_up + (h * UPW + r) * static_cast<int64_t>(KV) + c);
    }
    float4 kx1[RI], kx2[RI], qx1[RI], qx2[RI], rc1[RI], rc2[RI], rs1[RI], rs2[RI];
#pragma unroll
    for (int it = 0; it < RI; ++it) {
        const int u = tid + it * THREADS;
        const int row = u / QU, rc = row < L ? row : L - 1, i0 = 4 * (u % QU);
        const float* kr = rows + rc * p.proj_ts + p.kr_off + i0;
        const float* qr = rows + rc * p.proj_ts + p.q_off + h * HD + NOPE + i0;
        kx1[it] = *reinterpret_cast<const float4*>(kr);
        kx2[it] = *reinterpret_cast<const float4*>(kr + HALF);
        qx1[it] = *reinterpret_cast<const float4*>(qr);
        qx2[it] = *reinterpret_cast<const float4*>(qr + HALF);
        rc1[it] = *reinterpret_cast<const float4*>(p.cosine + rc * ROPE + i0);
        rc2[it] = *reinterpret_cast<const float4*>(p.cosine + rc * ROPE + i0 + HALF);
        rs1[it] = *reinterpret_cast<const float4*>(p.sine + rc * ROPE + i0);
        rs2[it] = *reinterpret_cast<const float4*>(p.sine + rc * ROPE + i0 + HALF);
    }
    float4 qn[NI];
#pragma unroll
    for (int it = 0; it < NI; ++it) {
        const int u = tid + it * THREADS;
        const int row = u / QN, rc = row < L ? row : L - 1;
        qn[it] = *reinterpret_cast<const float4*>(rows + rc * p.proj_ts + p.q_off + h * HD + 4 * (u % QN));
    }
    if constexpr (!LNIN) {
        const float4 wv = *reinterpret_cast<const float4*>(p.ln_w + 4 * lc);
        const float4 bv = p.ln_b ? *reinterpret_cast<const float4*>(p.ln_b + 4 * lc) : make_float4(0.f, 0.f, 0.f, 0.f);

        // LayerNorm of the latent rows into xq_s (bf16), the kv_up rows into wu_s.
        // The passes (rows) advance together, one reduction level at a time, so
        // that their cross-lane exchanges overlap; each row's arithmetic is that
        // of layer_norm_vec_kernel with 16 lanes per row.
        {
            const double inv_dim = 1.0 / static_cast<double>(KV);
            double mean[PASSES], sumsq[PASSES];  // the centred values are recomputed where used
#pragma unroll
            for (int ps = 0; ps < PASSES; ++ps) {
                const float4 x = xs[ps];
                mean[ps] = (static_cast<double>(x.x) + static_cast<double>(x.y)) +
                           (static_cast<double>(x.z) + static_cast<double>(x.w));
            }
            auto row_sums = [](double (&v)[PASSES]) {  // butterfly over the row's 16 lanes: xor 8, 4, 2, 1
#pragma unroll
                for (int ps = 0; ps < PASSES; ++ps) v[ps] += xor_row_d<8>(v[ps]);
#pragma unroll
                for (int ps = 0; ps < PASSES; ++ps) v[ps] += xor_row_d<4>(v[ps]);
#pragma unroll
                for (int ps = 0; ps < PASSES; ++ps) v[ps] += xor_row_d<2>(v[ps]);
#pragma unroll
                for (int ps = 0; ps < PASSES; ++ps) v[ps] += xor_row_d<1>(v[ps]);
            };
            row_sums(mean);
#pragma unroll
            for (int ps = 0; ps < PASSES; ++ps) {
                const float4 x = xs[ps];
                mean[ps] *= inv_dim;
                const double a0 = static_cast<double>(x.x) - mean[ps], a1 = static_cast<double>(x.y) - mean[ps];
                const double a2 = static_cast<double>(x.z) - mean[ps], a3 = static_cast<double>(x.w) - mean[ps];
                sumsq[ps] = (a0 * a0 + a1 * a1) + (a2 * a2 + a3 * a3);
            }
            row_sums(sumsq);
#pragma unroll
            for (int ps = 0; ps < PASSES; ++ps) {
                const int row = ps * (THREADS / 16) + lr;
                const float4 x = xs[ps];
                const double a0 = static_cast<double>(x.x) - mean[ps], a1 = static_cast<double>(x.y) - mean[ps];
                const double a2 = static_cast<double>(x.z) - mean[ps], a3 = static_cast<double>(x.w) - mean[ps];
                const double rstd = 1.0 / sqrt(fma(sumsq[ps], inv_dim, p.ln_eps));
                const bool active = row < L;
                const u16 o0 = active ? AttnElem<true>::from(static_cast<float>((a0 * rstd) * wv.x + static_cast<double>(bv.x))) : u16(0);
                const u16 o1 = active ? AttnElem<true>::from(static_cast<float>((a1 * rstd) * wv.y + static_cast<double>(bv.y))) : u16(0);
                const u16 o2 = active ? AttnElem<true>::from(static_cast<float>((a2 * rstd) * wv.z + static_cast<double>(bv.z))) : u16(0);
                const u16 o3 = active ? AttnElem<true>::from(static_cast<float>((a3 * rstd) * wv.w + static_cast<double>(bv.w))) : u16(0);
                *reinterpret_cast<uint2*>(xq_s + row * XP + 4 * lc) =
                    make_uint2(static_cast<uint32_t>(o0) | (static_cast<uint32_t>(o1) << 16),
                               static_cast<uint32_t>(o2) | (static_cast<uint32_t>(o3) << 16));
            }
        }
    }
#pragma unroll
    for (int it = 0; it < WUI; ++it) {
        const int u = tid + it * THREADS;
        if (u < WUN) {
            const int r = u / (KV / 8), c = (u % (KV / 8)) * 8;
            *reinterpret_cast<uint4*>(wu_s + r * XP + c) = wur[it];
        }
    }
    // 3. Rotated k_rope into k_s, four pairs per thread (rows beyond L: zero).
#pragma unroll
    for (int it = 0; it < RI; ++it) {
        const int u = tid + it * THREADS;
        const int row = u / QU, i0 = 4 * (u % QU);
        const float x1[4] = {kx1[it].x, kx1[it].y, kx1[it].z, kx1[it].w};
        const float x2[4] = {kx2[it].x, kx2[it].y, kx2[it].z, kx2[it].w};
        const float c1[4] = {rc1[it].x, rc1[it].y, rc1[it].z, rc1[it].w};
        const float c2[4] = {rc2[it].x, rc2[it].y, rc2[it].z, rc2[it].w};
        const float s1[4] = {rs1[it].x, rs1[it].y, rs1[it].z, rs1[it].w};
        const float s2[4] = {rs2[it].x, rs2[it].y, rs2[it].z, rs2[it].w};
        u16 o1[4], o2[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            rot(x1[j], x2[j], c1[j], s1[j], c2[j], s2[j], o1[j], o2[j]);
            if (row >= L) o1[j] = o2[j] = 0;
        }
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            k_s[row * KP + NOPE + i0 + j] = o1[j];
            k_s[row * KP + NOPE + i0 + j + HALF] = o2[j];
        }
    }
    __syncthreads();

    // 2. kv = LN(latent) . W_up^T for this head: k_nope into k_s, v transposed into vt_s.
    {
        constexpr int RT = LMAX / 16, CT = UPW / 16;
        for (int tix = wave; tix < RT * CT; tix += NW) {
            // LNIN: tile (w + NW j, ct) for j, ct in order; otherwise tiles w, w + NW, ... in row-major order.
            const int rt = LNIN ? wave + NW * (tix / (NW * CT)) : tix / CT;
            const int ct = LNIN ? (tix / NW) % CT : tix % CT;
            f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int ks = 0; ks < KV / 32; ++ks) {
                bf16x8 a;
                if constexpr (LNIN) {  // rows past L are zero, as the LayerNorm form stores them
                    a = __builtin_bit_cast(bf16x8, 16 * rt + li < L ? afr[tix / (NW * CT)][ks] : uint4{0u, 0u, 0u, 0u});
                } else {
                    a = __builtin_bit_cast(bf16x8, *reinterpret_cast<const uint4*>(xq_s + (16 * rt + li) * XP + 32 * ks + 8 * g));
                }
                const bf16x8 bw = __builtin_bit_cast(
                    bf16x8, *reinterpret_cast<const uint4*>(wu_s + (16 * ct + li) * XP + 32 * ks + 8 * g));
                acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, bw, acc, 0, 0, 0);
            }
            const int col = 16 * ct + li;
#pragma unroll
            for (int v = 0; v < 4; ++v) {
                const int row = 16 * rt + 4 * g + v;
                const u16 e = AttnElem<true>::from(acc[v]);
                if (col < NOPE) {
                    k_s[row * KP + col] = e;
                } else {
                    vt_s[(col - NOPE) * VP + row] = e;
                }
            }
        }
    }
    __syncthreads();  // xq_s (the latent) is free from here on
    // 4. q of this head over the latent: the nope part as loaded, the rope
    // part rotated (rows beyond L: zero).
#pragma unroll
    for (int it = 0; it < NI; ++it) {
        const int u = tid + it * THREADS;
        const int row = u / QN, q4 = u % QN;
        const float a4[4] = {qn[it].x, qn[it].y, qn[it].z, qn[it].w};
#pragma unroll
        for (int j = 0; j < 4; ++j) xq_s[row * KP + 4 * q4 + j] = row < L ? AttnElem<true>::from(a4[j]) : u16(0);
    }
#pragma unroll
    for (int it = 0; it < RI; ++it) {
        const int u = tid + it * THREADS;
        const int row = u / QU, i0 = 4 * (u % QU);
        const float a4[4] = {qx1[it].x, qx1[it].y, qx1[it].z, qx1[it].w};
        const float b4[4] = {qx2[it].x, qx2[it].y, qx2[it].z, qx2[it].w};
        const float c1[4] = {rc1[it].x, rc1[it].y, rc1[it].z, rc1[it].w};
        const float c2[4] = {rc2[it].x, rc2[it].y, rc2[it].z, rc2[it].w};
        const float s1[4] = {rs1[it].x, rs1[it].y, rs1[it].z, rs1[it].w};
        const float s2[4] = {rs2[it].x, rs2[it].y, rs2[it].z, rs2[it].w};
        u16 o1[4], o2[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            rot(a4[j], b4[j], c1[j], s1[j], c2[j], s2[j], o1[j], o2[j]);
            if (row >= L) o1[j] = o2[j] = 0;
        }
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            xq_s[row * KP + NOPE + i0 + j] = o1[j];
            xq_s[row * KP + NOPE + i0 + j + HALF] = o2[j];
        }
    }
    __syncthreads();

    // 5. Causal attention (top-left), keys and values from LDS, 64 keys per softmax step.
    int tiles[TPW];  // tile t and its mirror 2*NW-1-t balance the causal triangle
#pragma unroll
    for (int j = 0; j < TPW / 2; ++j) {
        tiles[2 * j] = wave + 2 * NW * j;
        tiles[2 * j + 1] = 2 * NW - 1 - wave + 2 * NW * j;
    }
    bf16x8 qb[TPW][HC];
    float m_run[TPW], l_run[TPW];
    f32x4 acc[TPW][OT];
#pragma unroll
    for (int i = 0; i < TPW; ++i) {
        const int q0 = 16 * tiles[i];
#pragma unroll
        for (int c = 0; c < HC; ++c) {
            qb[i][c] = __builtin_bit_cast(bf16x8, *reinterpret_cast<const uint4*>(xq_s + (q0 + li) * KP + 32 * c + 8 * g));
        }
        m_run[i] = -INFINITY;
        l_run[i] = 0.0f;
#pragma unroll
        for (int t = 0; t < OT; ++t) acc[i][t] = f32x4{0.f, 0.f, 0.f, 0.f};
    }
    for (int kbase = 0; kbase < L; kbase += kKeysPerChunk) {
#pragma unroll
        for (int i = 0; i < TPW; ++i) {
            const int q0 = 16 * tiles[i];
            if (q0 >= L || kbase > q0 + 15) continue;
            f32x4 sc[4];
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                sc[t] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int c = 0; c < HC; ++c) {
                    const bf16x8 a = __builtin_bit_cast(
                        bf16x8, *reinterpret_cast<const uint4*>(k_s + (kbase + 16 * t + li) * KP + 32 * c + 8 * g));
                    sc[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, qb[i][c], sc[t], 0, 0, 0);
                }
            }
            const int qpos = q0 + li;
            float mx = -INFINITY;
#pragma unroll
            for (int t = 0; t < 4; ++t) {
#pragma unroll
                for (int v = 0; v < 4; ++v) {
                    const int key = kbase + 16 * t + 4 * g + v;
                    const float x = (key < L && key <= qpos) ? (RAWMAX ? sc[t][v] : sc[t][v] * p.scale_log2) : -INFINITY;
                    sc[t][v] = x;
                    mx = fmaxf(mx, x);
                }
            }
            mx = xor_max(mx, 16);
            mx = xor_max(mx, 32);
            if constexpr (RAWMAX) mx *= p.scale_log2;  // the max of the scaled scores (the scale is positive)
            const float m_new = fmaxf(m_run[i], mx);
            const float m_use = m_new == -INFINITY ? 0.0f : m_new;
            const float corr = __builtin_amdgcn_exp2f(m_run[i] - m_use);
            m_run[i] = m_new;
            float psum = 0.0f;
#pragma unroll
            for (int t = 0; t < 4; ++t) {
#pragma unroll
                for (int v = 0; v < 4; ++v) {
                    const float e = __builtin_amdgcn_exp2f(RAWMAX ? fmaf(sc[t][v], p.scale_log2, -m_use) : sc[t][v] - m_use);
                    sc[t][v] = e;
                    psum += e;
                }
            }
            l_run[i] = l_run[i] * corr + psum;
#pragma unroll
            for (int t = 0; t < OT; ++t) {
#pragma unroll
                for (int v = 0; v < 4; ++v) acc[i][t][v] *= corr;
            }
#pragma unroll
            for (int half = 0; half < 2; ++half) {
                bf16x8 pb;
#pragma unroll
                for (int v = 0; v < 4; ++v) {
                    pb[v] = static_cast<__bf16>(sc[2 * half][v]);
                    pb[4 + v] = static_cast<__bf16>(sc[2 * half + 1][v]);
                }
#pragma unroll
                for (int t = 0; t < OT; ++t) {
                    const u16* vrow = vt_s + (16 * t + li) * VP + kbase + 32 * half + 4 * g;
                    const uint2 lo = *reinterpret_cast<const uint2*>(vrow);
                    const uint2 hi = *reinterpret_cast<const uint2*>(vrow + 16);
                    const uint4 raw = {lo.x, lo.y, hi.x, hi.y};
                    acc[i][t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, raw), pb, acc[i][t],
                                                                         0, 0, 0);
                }
            }
        }
    }
    // 6. Normalise and store [B, L, H, hd].
#pragma unroll
    for (int i = 0; i < TPW; ++i) {
        const int qi = 16 * tiles[i] + li;
        float l = xor_sum(l_run[i], 16);
        l = xor_sum(l, 32);
        if (qi >= L) continue;
        const float inv = 1.0f / l;
        float* orow = p.out + ((b * L + qi) * p.heads + h) * HD;
#pragma unroll
        for (int t = 0; t < OT; ++t) {
            *reinterpret_cast<float4*>(orow + 16 * t + 4 * g) =
                make_float4(acc[i][t][0] * inv, acc[i][t][1] * inv, acc[i][t][2] * inv, acc[i][t][3] * inv);
        }
    }
}

// ------------------------------------------------- whole MLA forward per window

// x of a window goes in MLK_MLA_XPARTS parts of K, MLK_MLA_XDEPTH of them in
// flight: one part at a time (its successor issued once it has landed) took
// the 256 x 128 workload from 30.6 to 29.5 us per step (median), because every
// block's part 0 then lands early instead of with the whole burst; four parts
// spill registers (37.5 us).
#ifndef MLK_MLA_XPARTS
#define MLK_MLA_XPARTS 2
#endif
#ifndef MLK_MLA_XDEPTH
#define MLK_MLA_XDEPTH 1
#endif

// mla_forward (montlok.cpp:1159-1211) for every causal query, one block of 8
// waves per window, so that neither the in_proj output nor the attention
// output goes through HBM: x is read once and the o_proj result written once.
//   in_proj  x (rounded to bf16) in LDS; wave w holds the W fragments of its
//            column tiles in registers (q nope and q rope of head w, plus
//            latent tile w for w < 4 or the k_rope tile for w = 4) and runs
//            them over the 8 row tiles: per (tile, row tile) the 8 k steps of
//            linear_tiles_kernel's chain, so the columns equal the separate
//            linear's bit for bit. Epilogue: q rounded to bf16 (its rope dims
//            rotated in fp64 first; the rope tiles take their W rows in an
//            order that puts each rotate_half pair in one lane), the latent
//            kept in fp32, k_rope rotated.
//   kv_norm  the LayerNorm of mla_attend_kernel (16 lanes per row, fp64),
//            into bf16.
//   heads    four at a time, two waves each: this head's kv_up rows, kv_up,
//            k = cat(k_nope, rope(k_rope)), causal attention, all as
//            mla_attend_kernel computes them (only the key tiles at or below
//            each query tile's diagonal); the normalised output rounded to
//            bf16 (the o_proj's operand) over the head's q columns.
//   o_proj   wave w: output tiles 2w, 2w + 1, W fragments in registers, the
//            attention output from LDS, the linear's chain again.
// The x / q / attention tile is [128 rows x 256] bf16 with 16-byte units
// XOR-swizzled by the row (unit u of row r at u ^ (r mod 8)), so the MFMA
// fragment reads (16 rows, one unit each per lane group) are conflict-free.
//
// PACKED: the three weights come re-laid in the kernel's fragment order
// (mla_pack_kernel), so that a wave's fragment load is one contiguous 1 KB
// read: in the row-major layout it touches 16 rows' 64-byte pieces, and with
// every block fetching the whole of each weight from L2 those loads bounded
// the kernel's start (in_proj fragments) and its last head round (o_proj
// fragments).
// Row order of the rope tiles: column 4g + v of a tile is rope dim 2g, 2g + 8,
// 2g + 1, 2g + 9 for v = 0..3, so a lane holds each dim with its
// rotate_half partner (dim +- 8).
__device__ __forceinline__ int mla_rope_order(int c) { return 2 * (c >> 2) + ((c >> 1) & 1) + 8 * (c & 1); }

// The packed weights of mla_window_kernel<H, true>, in 16-byte units (8 bf16):
// in_proj unit (tile * D / 32 + s) * 64 + lane holds W_in row 16 tile + r,
// k = 32 s + 8 (lane / 16) .. + 7, with r = lane % 16, or mla_rope_order of
// it for the rope tiles (each head's q rope tile 2h + 1 and the k_rope tile
// 2H + 4); then the kv_up rows, unit ((head * CT + ct) * KV / 32 + ks) * 64 +
// lane = row head * UPW + 16 ct + r, k = 32 ks + 8 (lane / 16); then the
// out_proj rows, unit (tile * D / 32 + s) * 64 + lane = row 16 tile + r.
template <int H>
struct MlaPack {
    static constexpr int HD = 32, NOPE = 16, ROPE = 16, KV = 64, D = H * HD, UPW = NOPE + HD, CT = UPW / 16;
    static constexpr int IN_TILES = (D + KV + ROPE) / 16;
    static constexpr int IN_UNITS = IN_TILES * (D / 32) * 64;
    static constexpr int UP_UNITS = H * CT * (KV / 32) * 64;
    static constexpr int OUT_UNITS = (D / 16) * (D / 32) * 64;
    static constexpr int UNITS = IN_UNITS + UP_UNITS + OUT_UNITS;
    __device__ static bool rope_tile(int tile) { return (tile < 2 * H && (tile & 1) != 0) || tile == 2 * H + KV / 16; }
    // The W_in row that lane row r of in_proj tile `tile` holds.
    __device__ static int in_row(int tile, int r) { return 16 * tile + (rope_tile(tile) ? mla_rope_order(r) : r); }
};

struct MlaWindowArgs {
    const float* x;  // [B, L, D], tokens x_ts apart, windows x_bs apart
    int64_t x_bs, x_ts;
    const u16* w_in;  // [D + KV + ROPE, D] bf16: q, kv_down, k_rope rows
    const float* ln_w;
    const float* ln_b;  // may be null
    double ln_eps;
    const u16* w_up;   // [H (NOPE + HD), KV] bf16
    const u16* w_out;  // [D, D] bf16
    const float* cosine;  // [L, ROPE]
    const float* sine;
    float* out;  // [B, L, D] contiguous
    int64_t length;
    float scale_log2;
};

template <int H, bool PACKED>
__global__ __launch_bounds__(512) void mla_window_kernel(MlaWindowArgs p) {
    constexpr int HD = 32, NOPE = 16, ROPE = 16, KV = 64;  // rope pairs (i, i + 8)
    constexpr int D = H * HD;
    constexpr int LMAX = 128, RT = LMAX / 16;
    constexpr int UPW = NOPE + HD;  // kv_up rows of one head
    constexpr int LP = KV + 8;      // latent pitch in bf16 elements (+16 bytes)
    constexpr int SLOT = 2 * LMAX * HD;  // one head's k [keys, HD] and v^T [HD, keys], bf16, swizzled
    constexpr int HG = 4;                // heads at a time, two waves each
    static_assert(H == 8, "the wave -> column tile map assumes 8 heads on 8 waves");
    static_assert(MlaPack<H>::HD == HD && MlaPack<H>::NOPE == NOPE && MlaPack<H>::ROPE == ROPE &&
                      MlaPack<H>::KV == KV && MlaPack<H>::UPW == UPW,
                  "the packed layout's geometry");
    __shared__ __attribute__((aligned(16))) u16 xq_s[LMAX * D];
    __shared__ __attribute__((aligned(16))) u16 lat_s[LMAX * LP];
    __shared__ __attribute__((aligned(16))) u16 kr_s[LMAX * ROPE];
    __shared__ __attribute__((aligned(16))) u16 head_s[HG * SLOT];
    __shared__ __attribute__((aligned(16))) float lnp_s[2 * KV];  // the LayerNorm's weight, then its bias (+0.0 if none)
    // [LMAX, KV] fp32 until the LayerNorm has run; 16-byte chunk c of row r at slot c ^ (r % 16), so the
    // epilogue's stores (16 rows, one chunk) and the LayerNorm's reads (one row, 16 chunks) are conflict-free.
    float* lat_f = reinterpret_cast<float*>(head_s);
    auto lat_at = [](int row, int chunk) { return row * KV + 4 * (chunk ^ (row & 15)); };

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int li = lane & 15;
    const int g = lane >> 4;
    const int L = static_cast<int>(p.length);
    const int64_t b = blockIdx.x;
    const float* xw = p.x + b * p.x_bs;
    // element (row, col) of the swizzled [LMAX, D] tile
    auto sw = [](int row, int col) { return row * D + ((((col >> 3) ^ (row & 7))) << 3) + (col & 7); };
    // The rope tiles (q rope of each head, k_rope) take their W rows in the order rp(c): column 4g + v of
    // the tile is rope dim 2g, 2g + 8, 2g + 1, 2g + 9 for v = 0..3, so the lane that holds a dim also
    // holds its rotate_half partner (dim +- 8). Each output element still comes from its own W row and x
    // row by the same chain of products, so the values are the linear's.
    auto rp = [](int c) { return mla_rope_order(c); };
    auto pack2 = [](float a, float b) -> uint32_t {  // two bf16 (round to nearest even) in one word
        return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2{a, b}, bf16x2));
    };

    // 1. Loads: x rows (rows past L read row L - 1 and are zeroed) and the W
    // fragments of this wave's in_proj tiles; everything else waits until
    // the W fragments are dead, so the registers hold.
    // x goes in XP parts of K (part q: k in [q D / XP, (q + 1) D / XP)), each followed by the W fragments of
    // its k steps. The first XDEPTH parts are issued here; part q + XDEPTH is issued once part q has landed
    // (after its barrier below), so that, with every block loading at once, the first parts land early and
    // their products run while the later parts arrive.
    constexpr int XP = MLK_MLA_XPARTS, XDEPTH = MLK_MLA_XDEPTH;
    static_assert(XP == 2 || XP == 4, "x in two or four parts of K");
    static_assert(XDEPTH >= 1 && XDEPTH <= XP, "parts in flight");
    constexpr int XU = LMAX * (D / 8) / 512;  // 8-float units per thread, XU / XP per part
    constexpr int SH = D / 32 / XP;           // k steps per part
    constexpr int PW = D / XP / 8;            // 8-float units of a row in one part
    constexpr int RU = XDEPTH * (XU / XP);    // registers hold the parts in flight: part q in slot q % XDEPTH
    float4 xa[RU], xb[RU];
    auto xunit = [&](int j, int& row, int& c8) {  // unit j: part j / (XU / XP), PW units per row
        const int q = j / (XU / XP), u = tid + 512 * (j % (XU / XP));
        row = u / PW;
        c8 = q * (D / XP) + (u % PW) * 8;
    };
    auto slot = [](int j) { return (j / (XU / XP)) % XDEPTH * (XU / XP) + j % (XU / XP); };
    auto load_x = [&](int q) {
#pragma unroll
        for (int j = q * (XU / XP); j < (q + 1) * (XU / XP); ++j) {
            int row, c8;
            xunit(j, row, c8);
            const float* src = xw + (row < L ? row : L - 1) * p.x_ts + c8;
            xa[slot(j)] = *reinterpret_cast<const float4*>(src);
            xb[slot(j)] = *reinterpret_cast<const float4*>(src + 4);
        }
    };
    const int tiles[3] = {2 * wave, 2 * wave + 1, 2 * H + (wave < 5 ? wave : 4)};
    const int wrow[3] = {li, rp(li), wave < 4 ? li : rp(li)};  // W row of lane li in each tile
    uint4 wf[3][D / 32];
#pragma unroll
    for (int q = 0; q < XP; ++q) {
        if (q < XDEPTH) load_x(q);
#pragma unroll
        for (int t = 0; t < 3; ++t)
#pragma unroll
            for (int s = q * SH; s < (q + 1) * SH; ++s)
                wf[t][s] = *reinterpret_cast<const uint4*>(
                    PACKED ? p.w_in + ((tiles[t] * (D / 32) + s) * 64 + lane) * 8
                           : p.w_in + (16 * tiles[t] + wrow[t]) * D + 32 * s + 8 * g);
    }
    // cos/sin of every row into LDS as doubles, converted once for all heads (the upper half of the head
    // slots, free until the heads run; the fp32 latent takes the lower half): thread t takes 4 values of
    // row t / 4 of both tables. A row of 16 doubles is 8 16-byte slots, pair p of the row at slot
    // p ^ (row % 8), so the 16 rows a fragment reads land in different banks.
    double* cs_d = reinterpret_cast<double*>(head_s + HG * SLOT / 2);  // [LMAX, ROPE] cos, then sin
    auto cs_at = [](int row, int pair) { return row * ROPE + 2 * (pair ^ (row & 7)); };
    static_assert(2 * LMAX * ROPE * 8 <= HG * SLOT, "rope tables in the upper half of the head slots");
    static_assert(LMAX * KV * 4 <= HG * SLOT, "the fp32 latent in the lower half");
    static_assert(LMAX * ROPE / 4 == 512, "one quad of each table per thread");
    const int crow = tid >> 2, ccol = 4 * (tid & 3), crc = crow < L ? crow : L - 1;
    const float4 cv = *reinterpret_cast<const float4*>(p.cosine + crc * ROPE + ccol);
    const float4 sv = *reinterpret_cast<const float4*>(p.sine + crc * ROPE + ccol);
    // The LayerNorm's weight and bias into LDS with the tables (read there after the epilogue instead of
    // from L2 then): threads 0 .. 2 KV / 4 - 1 take one float4 each. A missing bias reads the weight and
    // masks it to +0.0 bit-wise (a select here would become a branch around the load, and the branch a
    // wait for every load in flight).
    static_assert(2 * KV / 4 <= 512, "one float4 of the LayerNorm parameters per thread");
    const bool ln_part = tid < 2 * KV / 4, ln_bias = tid >= KV / 4;
    const uint32_t bmask = p.ln_b != nullptr || !ln_bias ? 0xffffffffu : 0u;
    const float* ln_src = ln_bias && p.ln_b != nullptr ? p.ln_b : p.ln_w;
    const float4 lnv = *reinterpret_cast<const float4*>(ln_src + 4 * ((ln_part ? tid : 0) % (KV / 4)));
    if (ln_part)
        *reinterpret_cast<float4*>(lnp_s + 4 * tid) =
            make_float4(__uint_as_float(__float_as_uint(lnv.x) & bmask), __uint_as_float(__float_as_uint(lnv.y) & bmask),
                        __uint_as_float(__float_as_uint(lnv.z) & bmask), __uint_as_float(__float_as_uint(lnv.w) & bmask));
    {
        const int p0 = ccol / 2;  // pairs p0, p0 + 1 of the row
        *reinterpret_cast<double2*>(cs_d + cs_at(crow, p0)) = make_double2(cv.x, cv.y);
        *reinterpret_cast<double2*>(cs_d + cs_at(crow, p0 + 1)) = make_double2(cv.z, cv.w);
        *reinterpret_cast<double2*>(cs_d + LMAX * ROPE + cs_at(crow, p0)) = make_double2(sv.x, sv.y);
        *reinterpret_cast<double2*>(cs_d + LMAX * ROPE + cs_at(crow, p0 + 1)) = make_double2(sv.z, sv.w);
    }

    // 2. in_proj: per (tile, row tile) the linear's chain over the 8 k steps, part by part of K. Waves 0..3
    // run their three tiles over every row tile; waves 4..7 their two q tiles over every row tile and the
    // k_rope tile over the two row tiles whose epilogue they take (w - 4 and w), into acc[2][0] and
    // acc[2][1].
    f32x4 acc[3][RT];
#pragma unroll
    for (int t = 0; t < 3; ++t)
#pragma unroll
        for (int m = 0; m < RT; ++m) acc[t][m] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int hf = 0; hf < XP; ++hf) {
#pragma unroll
        for (int j = hf * (XU / XP); j < (hf + 1) * (XU / XP); ++j) {
            int row, c8;
            xunit(j, row, c8);
            const bool live = row < L;
            const float4 a = xa[slot(j)], b4 = xb[slot(j)];
            const float v[8] = {a.x, a.y, a.z, a.w, b4.x, b4.y, b4.z, b4.w};
            bf16x8 o;
#pragma unroll
            for (int e = 0; e < 8; ++e) o[e] = static_cast<__bf16>(live ? v[e] : 0.0f);
            *reinterpret_cast<bf16x8*>(xq_s + sw(row, c8)) = o;
        }
        __syncthreads();
        if (hf + XDEPTH < XP) load_x(hf + XDEPTH);
        auto rows = [&](auto nt_c) {  // the first NT tiles over every row tile
            constexpr int NT = decltype(nt_c)::value;
#pragma unroll
            for (int m = 0; m < RT; ++m) {
#pragma unroll
                for (int s = hf * SH; s < (hf + 1) * SH; ++s) {
                    const bf16x8 xf = *reinterpret_cast<const bf16x8*>(xq_s + sw(16 * m + li, 32 * s + 8 * g));
#pragma unroll
                    for (int t = 0; t < NT; ++t)
                        acc[t][m] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, wf[t][s]), xf,
                                                                            acc[t][m], 0, 0, 0);
                }
            }
        };
        if (wave < 4) {
            rows(std::integral_constant<int, 3>{});
        } else {
            rows(std::integral_constant<int, 2>{});
#pragma unroll
            for (int u = 0; u < 2; ++u) {
                const int m = wave - 4 + 4 * u;
#pragma unroll
                for (int s = hf * SH; s < (hf + 1) * SH; ++s) {
                    const bf16x8 xf = *reinterpret_cast<const bf16x8*>(xq_s + sw(16 * m + li, 32 * s + 8 * g));
                    acc[2][u] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, wf[2][s]), xf,
                                                                        acc[2][u], 0, 0, 0);
                }
            }
        }
    }
    __syncthreads();  // every wave is done with x

    // 3. Epilogue: lane (g, li) of row tile m holds row 16 m + li, columns 4g .. 4g + 3 of each tile
    // (rope dims 2g, 2g + 8, 2g + 1, 2g + 9 in the rope tiles): q rounded to bf16, its rope dims rotated
    // first; the latent kept in fp32 (waves 0..3); k_rope rotated (waves 4..7 hold its tile; wave 4 + i
    // takes row tiles i and i + 4). rotate_half as rope_kernel: x1 c - x2 s on dims d < 8, x2 c + x1 s on
    // d + 8, two fp64 products and their sum rounded to fp64, then to fp32; the product of two floats is
    // exact in fp64, so the sum is one fma with the same result. Two things the separate operators do are
    // left out, as neither changes a stored output bit: the linear's zero bias, which only turns a -0
    // into +0 (a zero's sign is lost in the sums, maxima and LayerNorm that follow), and the zeroing of
    // rows past L (their x rows are zero; no stored query reads them as queries, and as keys they lie past
    // every stored query's diagonal).
    auto rope4 = [](const f32x4& y, const double2& ca, const double2& cb, const double2& sa, const double2& sb,
                    float (&o)[4]) {
        const double x0 = static_cast<double>(y[0]), x8 = static_cast<double>(y[1]);  // dims 2g, 2g + 8
        const double x1 = static_cast<double>(y[2]), x9 = static_cast<double>(y[3]);  // dims 2g + 1, 2g + 9
        o[0] = static_cast<float>(__fma_rn(x0, ca.x, -__dmul_rn(x8, sa.x)));
        o[1] = static_cast<float>(__fma_rn(x8, cb.x, __dmul_rn(x0, sb.x)));
        o[2] = static_cast<float>(__fma_rn(x1, ca.y, -__dmul_rn(x9, sa.y)));
        o[3] = static_cast<float>(__fma_rn(x9, cb.y, __dmul_rn(x1, sb.y)));
    };
#pragma unroll
    for (int m = 0; m < RT; ++m) {
        const int row = 16 * m + li;
        const f32x4 yn = acc[0][m], yr = acc[1][m], y3 = acc[2][m];
        const double2 ca = *reinterpret_cast<const double2*>(cs_d + cs_at(row, g));      // cos, dims 2g, 2g + 1
        const double2 cb = *reinterpret_cast<const double2*>(cs_d + cs_at(row, g + 4));  // dims 2g + 8, 2g + 9
        const double2 sa = *reinterpret_cast<const double2*>(cs_d + LMAX * ROPE + cs_at(row, g));
        const double2 sb = *reinterpret_cast<const double2*>(cs_d + LMAX * ROPE + cs_at(row, g + 4));
        float qr[4];
        rope4(yr, ca, cb, sa, sb, qr);
        const int q0 = HD * wave;
        *reinterpret_cast<uint2*>(xq_s + sw(row, q0 + 4 * g)) = make_uint2(pack2(yn[0], yn[1]), pack2(yn[2], yn[3]));
        *reinterpret_cast<uint32_t*>(xq_s + sw(row, q0 + NOPE + 2 * g)) = pack2(qr[0], qr[2]);
        *reinterpret_cast<uint32_t*>(xq_s + sw(row, q0 + NOPE + 2 * g + 8)) = pack2(qr[1], qr[3]);
        if (wave < 4) *reinterpret_cast<f32x4*>(lat_f + lat_at(row, 4 * wave + g)) = y3;
    }
    if (wave >= 4) {  // k_rope of row tiles w - 4 and w
#pragma unroll
        for (int u = 0; u < 2; ++u) {
            const int row = 16 * (wave - 4 + 4 * u) + li;
            const double2 ca = *reinterpret_cast<const double2*>(cs_d + cs_at(row, g));
            const double2 cb = *reinterpret_cast<const double2*>(cs_d + cs_at(row, g + 4));
            const double2 sa = *reinterpret_cast<const double2*>(cs_d + LMAX * ROPE + cs_at(row, g));
            const double2 sb = *reinterpret_cast<const double2*>(cs_d + LMAX * ROPE + cs_at(row, g + 4));
            float kr[4];
            rope4(acc[2][u], ca, cb, sa, sb, kr);
            *reinterpret_cast<uint32_t*>(kr_s + row * ROPE + 2 * g) = pack2(kr[0], kr[2]);
            *reinterpret_cast<uint32_t*>(kr_s + row * ROPE + 2 * g + 8) = pack2(kr[1], kr[3]);
        }
    }
    __syncthreads();
    // LayerNorm operands: four lanes per row, lane q = lane % 4 holding the row's four-column groups q,
    // q + 4, q + 8, q + 12; wave w takes rows 16 w .. 16 w + 15.
    const int lq = lane & 3, lrow = 16 * wave + (lane >> 2);
    float4 lnw[4], lnb[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        lnw[i] = *reinterpret_cast<const float4*>(lnp_s + 4 * (lq + 4 * i));
        lnb[i] = *reinterpret_cast<const float4*>(lnp_s + KV + 4 * (lq + 4 * i));
    }
    const int grp = wave >> 1;  // head group: heads grp, grp + HG
    const int wg = wave & 1;
    // The kv_up B fragments of the group's first head (lane (g, li): W_up row 16 ct + li, k = 32 ks + 8g ..),
    // in flight during the LayerNorm.
    constexpr int CT = UPW / 16;
    uint4 wu[CT][KV / 32];
#pragma unroll
    for (int ct = 0; ct < CT; ++ct)
#pragma unroll
        for (int ks = 0; ks < KV / 32; ++ks)
            wu[ct][ks] = *reinterpret_cast<const uint4*>(
                PACKED ? p.w_up + (((grp * CT + ct) * (KV / 32) + ks) * 64 + lane) * 8
                       : p.w_up + (grp * UPW + 16 * ct + li) * KV + 32 * ks + 8 * g);

    // 4. kv_norm: LayerNorm of the latent rows into bf16 with mla_attend_kernel's arithmetic: per group of
    // four columns (a + b) + (c + d) in fp64, the row's 16 groups combined by the butterfly xor 8, 4, 2, 1
    // over the groups. Lane q holds groups q, q + 4, q + 8, q + 12, so the xor-8 and xor-4 levels pair
    // groups inside the lane (each added in the butterfly's order, the own group first) and xor 2, xor 1
    // are exchanges inside the quad: every sum is formed exactly as the 16-lane form forms it.
    {
        const double inv_dim = 1.0 / static_cast<double>(KV);
        float4 xv[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) xv[i] = *reinterpret_cast<const float4*>(lat_f + lat_at(lrow, lq + 4 * i));
        auto row_sum = [](const double (&sg)[4]) {  // sg[i]: the sum of group lq + 4 i
            double u = (sg[0] + sg[2]) + (sg[1] + sg[3]);  // xor 8 (q with q + 8, q + 4 with q + 12), then xor 4
            u += xor_row_d<2>(u);
            u += xor_row_d<1>(u);
            return u;
        };
        double sg[4];
#pragma unroll
        for (int i = 0; i < 4; ++i)
            sg[i] = (static_cast<double>(xv[i].x) + static_cast<double>(xv[i].y)) +
                    (static_cast<double>(xv[i].z) + static_cast<double>(xv[i].w));
        const double mean = row_sum(sg) * inv_dim;
        double ac[4][4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            ac[i][0] = static_cast<double>(xv[i].x) - mean;
            ac[i][1] = static_cast<double>(xv[i].y) - mean;
            ac[i][2] = static_cast<double>(xv[i].z) - mean;
            ac[i][3] = static_cast<double>(xv[i].w) - mean;
            sg[i] = (ac[i][0] * ac[i][0] + ac[i][1] * ac[i][1]) + (ac[i][2] * ac[i][2] + ac[i][3] * ac[i][3]);
        }
        const double rstd = 1.0 / sqrt(fma(row_sum(sg), inv_dim, p.ln_eps));
        const uint32_t live = lrow < L ? 0xffffffffu : 0u;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const float o0 = static_cast<float>((ac[i][0] * rstd) * lnw[i].x + static_cast<double>(lnb[i].x));
            const float o1 = static_cast<float>((ac[i][1] * rstd) * lnw[i].y + static_cast<double>(lnb[i].y));
            const float o2 = static_cast<float>((ac[i][2] * rstd) * lnw[i].z + static_cast<double>(lnb[i].z));
            const float o3 = static_cast<float>((ac[i][3] * rstd) * lnw[i].w + static_cast<double>(lnb[i].w));
            *reinterpret_cast<uint2*>(lat_s + lrow * LP + 4 * (lq + 4 * i)) = make_uint2(pack2(o0, o1) & live, pack2(o2, o3) & live);
        }
    }
    __syncthreads();  // the fp32 latent is dead: the head slots take its place

    // 5. Heads, HG at a time, two waves each: group grp takes heads grp and grp + HG. Slot layouts
    // (16-byte units swizzled so the MFMA operand reads are conflict-free):
    //   k   [key][HD]   unit u of key r at u ^ ((r >> 1) & 3)
    //   v^T [HD][key]   unit u of dim d at u ^ (d & 7)
    u16* k_s = head_s + grp * SLOT;
    u16* vt_s = k_s + LMAX * HD;
    auto k_at = [](int key, int dim) { return key * HD + ((((dim >> 3) ^ ((key >> 1) & 3))) << 3) + (dim & 7); };
    auto v_at = [](int dim, int key) { return dim * LMAX + ((((key >> 3) ^ (dim & 7))) << 3) + (key & 7); };
    {  // the rotated k_rope, the same for every head, into the k rows (dims NOPE .. HD - 1) of every slot:
       // thread t copies row t % 128 into slot t / 128
        const int row = tid & (LMAX - 1);
        static_assert(512 == HG * LMAX, "one row of one slot per thread");
#pragma unroll
        for (int hf = 0; hf < 2; ++hf)
            *reinterpret_cast<uint4*>(head_s + (tid / LMAX) * SLOT + k_at(row, NOPE + 8 * hf)) =
                *reinterpret_cast<const uint4*>(kr_s + row * ROPE + 8 * hf);
    }
    uint4 wo[2][D / 32];  // o_proj fragments, fetched during the last round (the loop is unrolled, so
                          // their addresses are not held across it)
#pragma unroll
    for (int r = 0; r < H / HG; ++r) {
        const int h = r * HG + grp;
        // kv = LN(latent) . W_up^T for this head (row tiles wg, wg + 2, ...): k_nope into k_s, v^T into vt_s.
#pragma unroll
        for (int j = 0; j < RT / 2; ++j) {
            const int rt = 2 * j + wg;
            bf16x8 la[KV / 32];
#pragma unroll
            for (int ks = 0; ks < KV / 32; ++ks)
                la[ks] = *reinterpret_cast<const bf16x8*>(lat_s + (16 * rt + li) * LP + 32 * ks + 8 * g);
            // k_nope is formed transposed (W_up rows as the A operand), so that each lane holds four
            // consecutive dims of one key; v as keys x dims, four consecutive keys of one dim: either way
            // one 8-byte store per lane. The products and their order over k are the same either way.
#pragma unroll
            for (int ct = 0; ct < CT; ++ct) {
                f32x4 a = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int ks = 0; ks < KV / 32; ++ks)
                    a = ct == 0 ? __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, wu[ct][ks]), la[ks], a, 0, 0, 0)
                                : __builtin_amdgcn_mfma_f32_16x16x32_bf16(la[ks], __builtin_bit_cast(bf16x8, wu[ct][ks]), a, 0, 0, 0);
                const uint2 e = make_uint2(pack2(a[0], a[1]), pack2(a[2], a[3]));
                if (ct == 0) {
                    *reinterpret_cast<uint2*>(k_s + k_at(16 * rt + li, 4 * g)) = e;  // key 16 rt + li, dims 4g ..
                } else {
                    *reinterpret_cast<uint2*>(vt_s + v_at(16 * (ct - 1) + li, 16 * rt + 4 * g)) = e;  // keys 16 rt + 4g ..
                }
            }
        }
        if (r + 1 < H / HG) {  // the next head's fragments
#pragma unroll
            for (int ct = 0; ct < CT; ++ct)
#pragma unroll
                for (int ks = 0; ks < KV / 32; ++ks)
                    wu[ct][ks] = *reinterpret_cast<const uint4*>(
                        PACKED ? p.w_up + ((((h + HG) * CT + ct) * (KV / 32) + ks) * 64 + lane) * 8
                               : p.w_up + ((h + HG) * UPW + 16 * ct + li) * KV + 32 * ks + 8 * g);
        }
        __syncthreads();
        if (r + 1 == H / HG) {
#pragma unroll
            for (int t = 0; t < 2; ++t)
#pragma unroll
                for (int s = 0; s < D / 32; ++s)
                    wo[t][s] = *reinterpret_cast<const uint4*>(
                        PACKED ? p.w_out + (((2 * wave + t) * (D / 32) + s) * 64 + lane) * 8
                               : p.w_out + (16 * (2 * wave + t) + li) * D + 32 * s + 8 * g);
        }
        // Causal attention (top-left) of head h: query tiles (wg, 7 - wg, wg + 2, 5 - wg), 16 rows each,
        // against key chunk 0 (keys 0..63) and, for the tiles past row 63 when L > 64, chunk 1 (keys
        // 64..127). The wave's tiles are compile-time, so each (chunk, tile) pair runs only the 16-key tiles
        // at or below its diagonal, masks only the diagonal one, and the four tiles' chunk-0 chains are
        // straight-line code that interleaves. A key tile above the diagonal is all -inf in attn_kernel's
        // softmax: it adds nothing to the max, +0 to the sum and zero weights to P, so leaving it out
        // gives the same bits. Keys past L need no mask of their own: a query row below L sees keys up
        // to itself only, and rows past L are computed but not stored. The first chunk of a tile starts
        // from m = -inf, l = 0, o = 0, where attn_kernel's rescale multiplies zeros by zero. Every other
        // step is attn_kernel's (running max, exp2, rescale, P in bf16).
        auto attend = [&](auto wg_c) {
            constexpr int WG = decltype(wg_c)::value;
            constexpr int TQ = 4;
            constexpr int QT[TQ] = {WG, 7 - WG, WG + 2, 5 - WG};
            bf16x8 qb[TQ];
            float m_run[TQ], l_run[TQ];
            f32x4 o[TQ][HD / 16];
#pragma unroll
            for (int i = 0; i < TQ; ++i) {
                qb[i] = *reinterpret_cast<const bf16x8*>(xq_s + sw(16 * QT[i] + li, HD * h + 8 * g));
#pragma unroll
                for (int t = 0; t < HD / 16; ++t) o[i][t] = f32x4{0.f, 0.f, 0.f, 0.f};
            }
            auto chunk = [&](auto kc_c, auto i_c) {
                constexpr int KC = decltype(kc_c)::value, I = decltype(i_c)::value;
                constexpr int DIAG = QT[I] - 4 * KC;              // the diagonal key tile (none when >= 4)
                constexpr int NKT = DIAG + 1 < 4 ? DIAG + 1 : 4;  // key tiles at or below the diagonal
                constexpr bool FIRST = KC == 0;
                static_assert(NKT >= 1, "a chunk with no key at or below the diagonal is not run");
                const int kbase = kKeysPerChunk * KC;
                f32x4 sc[NKT];
#pragma unroll
                for (int t = 0; t < NKT; ++t) {
                    const bf16x8 ka = *reinterpret_cast<const bf16x8*>(k_s + k_at(kbase + 16 * t + li, 8 * g));
                    sc[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ka, qb[I], f32x4{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
                }
                float mx = -INFINITY;
#pragma unroll
                for (int t = 0; t < NKT; ++t) {
#pragma unroll
                    for (int v = 0; v < 4; ++v) {
                        float xv = sc[t][v];
                        if (t == DIAG) xv = 4 * g + v <= li ? xv : -INFINITY;  // key 16 t + 4g + v <= query li
                        sc[t][v] = xv;
                        mx = fmaxf(mx, xv);
                    }
                }
                mx = fmaxf(mx, lane_xor16(mx));
                mx = fmaxf(mx, lane_xor32(mx));
                mx *= p.scale_log2;  // the max of the scaled scores (the scale is positive)
                const float m_new = FIRST ? mx : fmaxf(m_run[I], mx);
                const float m_use = m_new == -INFINITY ? 0.0f : m_new;
                float corr = 0.0f;
                if constexpr (!FIRST) corr = __builtin_amdgcn_exp2f(m_run[I] - m_use);
                m_run[I] = m_new;
                float psum = 0.0f;
#pragma unroll
                for (int t = 0; t < NKT; ++t) {
#pragma unroll
                    for (int v = 0; v < 4; ++v) {
                        const float e = __builtin_amdgcn_exp2f(fmaf(sc[t][v], p.scale_log2, -m_use));
                        sc[t][v] = e;
                        psum += e;
                    }
                }
                if constexpr (FIRST) {
                    l_run[I] = psum;
                } else {
                    l_run[I] = l_run[I] * corr + psum;
#pragma unroll
                    for (int t = 0; t < HD / 16; ++t) {
#pragma unroll
                        for (int v = 0; v < 4; ++v) o[I][t][v] *= corr;
                    }
                }
#pragma unroll
                for (int half = 0; half < 2; ++half) {
                    if (2 * half >= NKT) continue;  // P is zero over both key tiles (known at compile time)
                    const int ta = 2 * half, tb = 2 * half + 1 < NKT ? 2 * half + 1 : ta;
                    const uint2 pa = make_uint2(pack2(sc[ta][0], sc[ta][1]), pack2(sc[ta][2], sc[ta][3]));
                    const uint2 pz = 2 * half + 1 < NKT ? make_uint2(pack2(sc[tb][0], sc[tb][1]), pack2(sc[tb][2], sc[tb][3]))
                                                        : make_uint2(0u, 0u);
                    const bf16x8 pb = __builtin_bit_cast(bf16x8, uint4{pa.x, pa.y, pz.x, pz.y});
#pragma unroll
                    for (int t = 0; t < HD / 16; ++t) {
                        const int dim = 16 * t + li, key0 = kbase + 32 * half + 4 * g;
                        const uint2 lo = *reinterpret_cast<const uint2*>(vt_s + v_at(dim, key0));
                        const uint2 hi = *reinterpret_cast<const uint2*>(vt_s + v_at(dim, key0 + 16));
                        const uint4 raw = {lo.x, lo.y, hi.x, hi.y};
                        o[I][t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, raw), pb, o[I][t],
                                                                           0, 0, 0);
                    }
                }
            };
            static_assert(LMAX == 2 * kKeysPerChunk, "two key chunks");
            using C0 = std::integral_constant<int, 0>;
            using C1 = std::integral_constant<int, 1>;
            chunk(C0{}, C0{});
            chunk(C0{}, C1{});
            chunk(C0{}, std::integral_constant<int, 2>{});
            chunk(C0{}, std::integral_constant<int, 3>{});
            if (L > kKeysPerChunk) {  // tiles 7 - wg and 5 - wg reach past key 63
                chunk(C1{}, C1{});
                chunk(C1{}, std::integral_constant<int, 3>{});
            }
            // Normalised output, rounded to bf16 as the o_proj takes it, over this head's q columns.
#pragma unroll
            for (int i = 0; i < TQ; ++i) {
                const int qi = 16 * QT[i] + li;
                float l = l_run[i] + lane_xor16(l_run[i]);
                l = l + lane_xor32(l);
                if (qi >= L) continue;
                const float inv = 1.0f / l;
#pragma unroll
                for (int t = 0; t < HD / 16; ++t) {
                    *reinterpret_cast<uint2*>(xq_s + sw(qi, HD * h + 16 * t + 4 * g)) =
                        make_uint2(pack2(o[i][t][0] * inv, o[i][t][1] * inv), pack2(o[i][t][2] * inv, o[i][t][3] * inv));
                }
            }
        };
        if (wg == 0) {
            attend(std::integral_constant<int, 0>{});
        } else {
            attend(std::integral_constant<int, 1>{});
        }
        __syncthreads();
    }

    // 6. o_proj: wave w computes output columns 32 w .. 32 w + 31 of every row, two row tiles at a time:
    // their 16 attention fragments are read first, then the four accumulation chains (two row tiles x two
    // column tiles, each the linear's chain over the 8 k steps) run interleaved.
    float* orow0 = p.out + b * static_cast<int64_t>(L) * D;
#pragma unroll
    for (int m = 0; m < RT; m += 2) {
        bf16x8 af[2][D / 32];
#pragma unroll
        for (int mm = 0; mm < 2; ++mm)
#pragma unroll
            for (int s = 0; s < D / 32; ++s)
                af[mm][s] = *reinterpret_cast<const bf16x8*>(xq_s + sw(16 * (m + mm) + li, 32 * s + 8 * g));
        f32x4 y[2][2];
#pragma unroll
        for (int mm = 0; mm < 2; ++mm)
#pragma unroll
            for (int t = 0; t < 2; ++t) y[mm][t] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int s = 0; s < D / 32; ++s)
#pragma unroll
            for (int mm = 0; mm < 2; ++mm)
#pragma unroll
                for (int t = 0; t < 2; ++t)
                    y[mm][t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, wo[t][s]), af[mm][s],
                                                                       y[mm][t], 0, 0, 0);
#pragma unroll
        for (int mm = 0; mm < 2; ++mm) {
            const int row = 16 * (m + mm) + li;
            if (row < L) {
#pragma unroll
                for (int t = 0; t < 2; ++t) {
                    *reinterpret_cast<f32x4*>(orow0 + row * D + HD * wave + 16 * t + 4 * g) =
                        y[mm][t] + f32x4{0.f, 0.f, 0.f, 0.f};
                }
            }
        }
    }
}


// ------------------------------------- whole MLA forward per span of 64 queries

// The k_rope tiles of mla_span_kernel take their W rows in this order: column c
// of tile tt (0, 1) is rope dim 2 (c / 4) + (c / 2) % 2 + 8 tt, plus 16 for odd
// c, so the lane holding dim i < 16 also holds its rotate_half partner i + 16.
__device__ __forceinline__ int mla_span_kr_dim(int c, int tt) { return 2 * (c >> 2) + ((c >> 1) & 1) + 8 * tt + 16 * (c & 1); }

// The packed weights of mla_span_kernel<true>, in 16-byte units (8 bf16), the
// order its waves load them: in_proj unit (tile * D / 32 + s) * 64 + lane holds
// W_in row in_row(tile, lane % 16), k = 32 s + 8 (lane / 16) .. + 7 (tiles: q
// 0..15, latent 16..19, k_rope 20, 21); then the kv_up rows, unit ((head * CT +
// ct) * KV / 32 + ks) * 64 + lane = row head * UPW + 16 ct + lane % 16; then the
// out_proj rows like the in_proj's.
struct MlaSpanPack {
    static constexpr int H = 4, HD = 64, NOPE = 32, ROPE = 32, KV = 64, D = H * HD, UPW = NOPE + HD, CT = UPW / 16;
    static constexpr int KR_T = (D + KV) / 16;
    static constexpr int IN_TILES = (D + KV + ROPE) / 16;
    static constexpr int IN_UNITS = IN_TILES * (D / 32) * 64;
    static constexpr int UP_UNITS = H * CT * (KV / 32) * 64;
    static constexpr int OUT_UNITS = (D / 16) * (D / 32) * 64;
    static constexpr int UNITS = IN_UNITS + UP_UNITS + OUT_UNITS;
    __device__ static int in_row(int tile, int r) { return tile >= KR_T ? D + KV + mla_span_kr_dim(r, tile - KR_T) : 16 * tile + r; }
};

// mla_forward (montlok.cpp:1159-1211) for every causal query at d_model 256,
// 4 heads of 64 (rope 32, nope 32), kv rank 64 and L <= 256: one block of 8
// waves per (window, span of 64 query rows), so that neither the in_proj
// output nor the attention output goes through HBM. A window's rows do not
// fit one block's LDS as keys and queries at once (mla_window_kernel's form),
// so each block walks the key rows in 64-row tiles up to its own span:
//   q        x of the span (bf16 in LDS); wave w: head w / 2, its nope
//            (w even) or rope (w odd) column tiles over the 4 row tiles, the
//            linear's chain over the 8 k steps; q rounded to bf16, its rope
//            dims rotated in fp64 first (the two rope tiles of a head sit in
//            one wave, so a lane holds dim i and its rotate_half partner
//            i + 16).
//   key tile t = 0 .. span: x rows of the tile (loaded a phase ahead), the
//            latent and k_rope columns of the in_proj (the same chains),
//            k_rope rotated into every head's k rows, the latent's LayerNorm
//            (mla_window_kernel's four lanes per row: layer_norm_vec_kernel's
//            sums), kv_up (wave w: head w / 2, three of its six column
//            tiles over the 4 row tiles), and the causal
//            attention of the span's queries against the tile with the
//            running max, sum and output carried across tiles: per query row
//            the chunk sequence of mla_attend_kernel (its 64-key chunks are
//            these tiles, in the same order), the same products and the same
//            softmax arithmetic, so the result is the four-launch path's bit
//            for bit. Wave w: head w / 2, query tiles (0, 3) or (1, 2) (the
//            diagonal tile's work balanced).
//   o_proj   the normalised output rounded to bf16 (the o_proj's operand)
//            in LDS, then wave w's two output column tiles over the 4 row
//            tiles, the linear's chain again.
// Blocks of one window run on one XCD (its L2 serves the later spans' reads
// of the window's x). PACKED: the three weights in MlaSpanPack's order, each
// wave's fragment load one contiguous 1 KB.
template <bool PACKED>
__global__ __launch_bounds__(512) void mla_span_kernel(MlaWindowArgs p, int spans) {
    using PK = MlaSpanPack;
    constexpr int H = 4, HD = 64, NOPE = 32, ROPE = 32, HALF = ROPE / 2, KV = 64, D = H * HD;
    constexpr int SPAN = 64, RT = SPAN / 16;  // rows per span and per key tile, 16-row tiles
    constexpr int UPW = NOPE + HD;            // kv_up rows of one head
    constexpr int LP = KV + 8;                // normalised latent pitch in bf16 elements (+16 bytes)
    constexpr int LAT_T = D / 16, KR_T = LAT_T + KV / 16;  // in_proj tiles: q 0 .., latent LAT_T .., k_rope KR_T ..
    // x of one row tile set, later the attention output: [SPAN, D] bf16, 16-byte unit u of row r at
    // u ^ (r % 8); q of the span in the same layout.
    __shared__ __attribute__((aligned(16))) u16 x_s[SPAN * D];
    __shared__ __attribute__((aligned(16))) u16 q_s[SPAN * D];
    // Per head: k [key][HD], unit u of key r at u ^ ((r / 2) % 8); v^T [HD][key], unit u of dim d at
    // u ^ ((d / 2) % 8): the 16 rows a fragment read touches land in distinct banks. The fp32 latent
    // ([SPAN, KV], 16-byte chunk c of row r at c ^ (r % 16)) lives in the v^T slots until kv_up.
    __shared__ __attribute__((aligned(16))) u16 k_s[H * SPAN * HD];
    __shared__ __attribute__((aligned(16))) u16 vt_s[H * HD * SPAN];
    __shared__ __attribute__((aligned(16))) u16 lat_s[SPAN * LP];
    __shared__ __attribute__((aligned(16))) float lnp_s[2 * KV];  // the LayerNorm's weight, then its bias
    __shared__ __attribute__((aligned(16))) float csq_s[2 * SPAN * ROPE];  // cos, then sin, of the span's rows
    static_assert(SPAN * KV * 4 <= H * HD * SPAN * 2, "the fp32 latent fits the v^T slots");
    float* lat_f = reinterpret_cast<float*>(vt_s);
    auto lat_at = [](int row, int chunk) { return row * KV + 4 * (chunk ^ (row & 15)); };
    auto sw = [](int row, int col) { return row * D + ((((col >> 3) ^ (row & 7))) << 3) + (col & 7); };
    auto k_at = [](int key, int dim) { return key * HD + ((((dim >> 3) ^ ((key >> 1) & 7))) << 3) + (dim & 7); };
    auto v_at = [](int dim, int key) { return dim * SPAN + ((((key >> 3) ^ ((dim >> 1) & 7))) << 3) + (key & 7); };
    auto pack2 = [](float a, float b) -> uint32_t {
        return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2{a, b}, bf16x2));
    };
    // rotate_half as rope_kernel: x1 c1 - x2 s1 on dim i, x2 c2 + x1 s2 on dim i + HALF, fp64 products
    // and sum, rounded to fp32.
    auto rope4 = [](const f32x4& x1, const f32x4& x2, const float4& c1, const float4& c2, const float4& s1,
                    const float4& s2, float (&o1)[4], float (&o2)[4]) {
        const float c1a[4] = {c1.x, c1.y, c1.z, c1.w}, c2a[4] = {c2.x, c2.y, c2.z, c2.w};
        const float s1a[4] = {s1.x, s1.y, s1.z, s1.w}, s2a[4] = {s2.x, s2.y, s2.z, s2.w};
#pragma unroll
        for (int v = 0; v < 4; ++v) {
            const double a = static_cast<double>(x1[v]), bq = static_cast<double>(x2[v]);
            o1[v] = static_cast<float>(__dsub_rn(__dmul_rn(a, c1a[v]), __dmul_rn(bq, s1a[v])));
            o2[v] = static_cast<float>(__dadd_rn(__dmul_rn(bq, c2a[v]), __dmul_rn(a, s2a[v])));
        }
    };

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int li = lane & 15;
    const int g = lane >> 4;
    const int L = static_cast<int>(p.length);
    const int64_t windows = gridDim.x / spans;
    int64_t b;
    int j;
    {
        const int64_t id = blockIdx.x;
        // The spans of a window are adjacent in dispatch order, in an order rotated from window to window:
        // consecutive blocks go to the shader arrays in turn, so each array gets heavy and light spans alike.
        int64_t wi, r;
        if (windows % 8 == 0) {  // XCD x = id % 8 takes windows x, x + 8, ...
            const int64_t k = id / 8;
            wi = k / spans;
            r = k % spans;
            b = id % 8 + 8 * wi;
        } else {
            wi = id / spans;
            r = id % spans;
            b = wi;
        }
        j = spans - 1 - static_cast<int>((r + wi) % spans);
    }
    const float* xw = p.x + b * p.x_bs;

    // x rows 64 t .. 64 t + 63 (rows past L read row L - 1, zeroed when stored): thread t takes 8-float
    // units t + 512 i, row u / 32.
    float4 xa[4], xb[4];
    auto load_x = [&](int t) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int u = tid + 512 * i, row = SPAN * t + u / 32;
            const float* src = xw + static_cast<int64_t>(row < L ? row : L - 1) * p.x_ts + (u % 32) * 8;
            xa[i] = *reinterpret_cast<const float4*>(src);
            xb[i] = *reinterpret_cast<const float4*>(src + 4);
        }
    };
    auto store_x = [&](int t) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int u = tid + 512 * i, r = u / 32;
            const bool live = SPAN * t + r < L;
            const float v[8] = {xa[i].x, xa[i].y, xa[i].z, xa[i].w, xb[i].x, xb[i].y, xb[i].z, xb[i].w};
            bf16x8 o;
#pragma unroll
            for (int e = 0; e < 8; ++e) o[e] = static_cast<__bf16>(live ? v[e] : 0.0f);
            *reinterpret_cast<bf16x8*>(x_s + sw(r, (u % 32) * 8)) = o;
        }
    };
    auto w_in_frag = [&](int tile, int s) {  // W_in row PK::in_row(tile, li), k = 32 s + 8 g .. + 7
        return *reinterpret_cast<const uint4*>(PACKED ? p.w_in + ((tile * (D / 32) + s) * 64 + lane) * 8
                                                      : p.w_in + PK::in_row(tile, li) * D + 32 * s + 8 * g);
    };

    // 1. q of the span.
    const int h = wave >> 1, wg = wave & 1;
    load_x(j);
    uint4 wq[2][D / 32];
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int s = 0; s < D / 32; ++s) wq[t][s] = w_in_frag(4 * h + 2 * wg + t, s);
    {  // the LayerNorm's weight and bias (+0.0 where there is none), as mla_window_kernel takes them
        const bool ln_part = tid < 2 * KV / 4, ln_bias = tid >= KV / 4;
        const uint32_t bmask = p.ln_b != nullptr || !ln_bias ? 0xffffffffu : 0u;
        const float* ln_src = ln_bias && p.ln_b != nullptr ? p.ln_b : p.ln_w;
        const float4 lnv = *reinterpret_cast<const float4*>(ln_src + 4 * ((ln_part ? tid : 0) % (KV / 4)));
        if (ln_part)
            *reinterpret_cast<float4*>(lnp_s + 4 * tid) =
                make_float4(__uint_as_float(__float_as_uint(lnv.x) & bmask), __uint_as_float(__float_as_uint(lnv.y) & bmask),
                            __uint_as_float(__float_as_uint(lnv.z) & bmask), __uint_as_float(__float_as_uint(lnv.w) & bmask));
    }
    {  // cos/sin rows of the span for the q rotation: thread t takes float4 t and t + 512 of [2, SPAN, ROPE]
#pragma unroll
        for (int k = 0; k < 2; ++k) {
            const int f = tid + 512 * k, tab = f / (SPAN * ROPE / 4), rem = f % (SPAN * ROPE / 4);
            const int row = rem / (ROPE / 4), pos = SPAN * j + row, pc = pos < L ? pos : L - 1;
            const float* src = (tab == 0 ? p.cosine : p.sine) + pc * ROPE + 4 * (rem % (ROPE / 4));
            *reinterpret_cast<float4*>(csq_s + 4 * f) = *reinterpret_cast<const float4*>(src);
        }
    }
    store_x(j);
    __syncthreads();
    load_x(0);  // key tile 0, stored once the q products are done
    // The weights of the key-tile loop, the same for every tile, fetched once and held: waves 0..3 the W_in
    // rows of latent tile w (run over the 4 row tiles); waves 4..7 one of the two k_rope tiles, RT_K =
    // (w - 4) / 2, over row tiles 2 ((w - 4) % 2) and the next. The k_rope tiles take their W rows in the
    // order mla_span_kr_dim(c): column 4g + v of tile T is rope dim 2g + 8T, + 16, 2g + 1 + 8T, + 16 for v = 0..3,
    // so a lane holds each dim i < 16 with its rotate_half partner i + 16 (each column still comes from its
    // own W row and x row by the linear's chain).
    constexpr int CT = UPW / 16, CTW = CT / 2;
    const int kt_t = (wave - 4) >> 1, kt_r = 2 * ((wave - 4) & 1);  // k_rope waves: tile, first row tile
    static_assert(PK::KR_T == KR_T && PK::D == D && PK::KV == KV && PK::UPW == UPW, "the packed layout's geometry");
    uint4 wl[D / 32];
#pragma unroll
    for (int s = 0; s < D / 32; ++s) wl[s] = w_in_frag(wave < 4 ? LAT_T + wave : KR_T + kt_t, s);

    {
        f32x4 aq[2][RT];
#pragma unroll
        for (int t = 0; t < 2; ++t)
#pragma unroll
            for (int m = 0; m < RT; ++m) aq[t][m] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int m = 0; m < RT; ++m)
#pragma unroll
            for (int s = 0; s < D / 32; ++s) {
                const bf16x8 xf = *reinterpret_cast<const bf16x8*>(x_s + sw(16 * m + li, 32 * s + 8 * g));
#pragma unroll
                for (int t = 0; t < 2; ++t)
                    aq[t][m] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, wq[t][s]), xf, aq[t][m],
                                                                       0, 0, 0);
            }
        // Lane (g, li) of row tile m holds row 16 m + li, columns 4g .. 4g + 3 of each tile.
        if (wg == 0) {
#pragma unroll
            for (int m = 0; m < RT; ++m)
#pragma unroll
                for (int t = 0; t < 2; ++t)
                    *reinterpret_cast<uint2*>(q_s + sw(16 * m + li, HD * h + 16 * t + 4 * g)) =
                        make_uint2(pack2(aq[t][m][0], aq[t][m][1]), pack2(aq[t][m][2], aq[t][m][3]));
        } else {
#pragma unroll
            for (int m = 0; m < RT; ++m) {
                const float* cr = csq_s + (16 * m + li) * ROPE + 4 * g;
                const float* sr = cr + SPAN * ROPE;
                float o1[4], o2[4];
                rope4(aq[0][m], aq[1][m], *reinterpret_cast<const float4*>(cr), *reinterpret_cast<const float4*>(cr + HALF),
                      *reinterpret_cast<const float4*>(sr), *reinterpret_cast<const float4*>(sr + HALF), o1, o2);
                *reinterpret_cast<uint2*>(q_s + sw(16 * m + li, HD * h + NOPE + 4 * g)) =
                    make_uint2(pack2(o1[0], o1[1]), pack2(o1[2], o1[3]));
                *reinterpret_cast<uint2*>(q_s + sw(16 * m + li, HD * h + NOPE + HALF + 4 * g)) =
                    make_uint2(pack2(o2[0], o2[1]), pack2(o2[2], o2[3]));
            }
        }
    }
    __syncthreads();  // q is in LDS; every wave is done with x

    // Attention state of the wave's two query tiles QT(i) = (wg, 3 - wg)[i] of head h.
    float m_run[2], l_run[2];
    f32x4 o[2][HD / 16];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int t = 0; t < HD / 16; ++t) o[i][t] = f32x4{0.f, 0.f, 0.f, 0.f};

    for (int t = 0; t <= j; ++t) {
        // The lane's row and group indices made opaque to the compiler per key tile, so the many LDS
        // addresses derived from them are formed where used instead of being held across the loop.
        int lane_t = lane;
        asm volatile("" : "+v"(lane_t));
        const int li = lane_t & 15;
        const int g = lane_t >> 4;
        // 2. x of key tile t into LDS (the k_rope waves' cos/sin in flight meanwhile: dims 2g + 8T, + 1 and
        // their partners + 16, of the two rows the lane rotates).
        float2 kcs[2][4];
        if (wave >= 4) {
#pragma unroll
            for (int u = 0; u < 2; ++u) {
                const int pos = SPAN * t + 16 * (kt_r + u) + li, pc = pos < L ? pos : L - 1;
                const float* cr = p.cosine + pc * ROPE + 2 * g + 8 * kt_t;
                const float* sr = p.sine + pc * ROPE + 2 * g + 8 * kt_t;
                kcs[u][0] = *reinterpret_cast<const float2*>(cr);
                kcs[u][1] = *reinterpret_cast<const float2*>(cr + HALF);
                kcs[u][2] = *reinterpret_cast<const float2*>(sr);
                kcs[u][3] = *reinterpret_cast<const float2*>(sr + HALF);
            }
        }
        // The kv_up B fragments of head h, column tiles 3 wg .. 3 wg + 2 (lane (g, li): W_up row
        // h UPW + 16 ct + li, k = 32 ks + 8g ..), in flight until step 5.
        uint4 wu[CTW][KV / 32];
#pragma unroll
        for (int c = 0; c < CTW; ++c)
#pragma unroll
            for (int ks = 0; ks < KV / 32; ++ks)
                wu[c][ks] = *reinterpret_cast<const uint4*>(
                    PACKED ? p.w_up + (((h * CT + CTW * wg + c) * (KV / 32) + ks) * 64 + lane) * 8
                           : p.w_up + (h * UPW + 16 * (CTW * wg + c) + li) * KV + 32 * ks + 8 * g);
        store_x(t);
        __syncthreads();  // x of tile t is in LDS; the previous tile's attention is done
        if (t < j) load_x(t + 1);  // the next tile's x, in flight until the next step 2
        // 3. Latent and k_rope columns of the tile's rows, each (tile, row tile) the linear's chain.
        if (wave < 4) {
            f32x4 al[RT];
#pragma unroll
            for (int m = 0; m < RT; ++m) al[m] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int s = 0; s < D / 32; ++s)
#pragma unroll
                for (int m = 0; m < RT; ++m) {
                    const bf16x8 xf = *reinterpret_cast<const bf16x8*>(x_s + sw(16 * m + li, 32 * s + 8 * g));
                    al[m] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, wl[s]), xf, al[m], 0, 0, 0);
                }
#pragma unroll
            for (int m = 0; m < RT; ++m) *reinterpret_cast<f32x4*>(lat_f + lat_at(16 * m + li, 4 * wave + g)) = al[m];
        } else {  // k_rope, rotated, into every head's k rows (dims NOPE ..)
            f32x4 a[2] = {f32x4{0.f, 0.f, 0.f, 0.f}, f32x4{0.f, 0.f, 0.f, 0.f}};
#pragma unroll
            for (int s = 0; s < D / 32; ++s)
#pragma unroll
                for (int u = 0; u < 2; ++u) {
                    const bf16x8 xf = *reinterpret_cast<const bf16x8*>(x_s + sw(16 * (kt_r + u) + li, 32 * s + 8 * g));
                    a[u] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, wl[s]), xf, a[u], 0, 0, 0);
                }
#pragma unroll
            for (int u = 0; u < 2; ++u) {
                const int row = 16 * (kt_r + u) + li;
                // a[u][0], a[u][2]: dims i = 2g + 8T and i + 1; a[u][1], a[u][3]: their partners i + 16, i + 17.
                const float2 c1 = kcs[u][0], c2 = kcs[u][1], s1 = kcs[u][2], s2 = kcs[u][3];
                const f32x4 x1 = {a[u][0], a[u][2], 0.f, 0.f}, x2 = {a[u][1], a[u][3], 0.f, 0.f};
                float o1[4], o2[4];
                rope4(x1, x2, make_float4(c1.x, c1.y, 0.f, 0.f), make_float4(c2.x, c2.y, 0.f, 0.f),
                      make_float4(s1.x, s1.y, 0.f, 0.f), make_float4(s2.x, s2.y, 0.f, 0.f), o1, o2);
                const uint32_t e1 = pack2(o1[0], o1[1]), e2 = pack2(o2[0], o2[1]);
#pragma unroll
                for (int hh = 0; hh < H; ++hh) {
                    *reinterpret_cast<uint32_t*>(k_s + hh * SPAN * HD + k_at(row, NOPE + 2 * g + 8 * kt_t)) = e1;
                    *reinterpret_cast<uint32_t*>(k_s + hh * SPAN * HD + k_at(row, NOPE + HALF + 2 * g + 8 * kt_t)) = e2;
                }
            }
        }
        __syncthreads();  // the fp32 latent and the rotated k_rope are in LDS; x is free

        // 4. kv_norm: waves 0..3, four lanes per row (lane q holds the row's four-column groups q, q + 4,
        // q + 8, q + 12; the butterfly's xor-8 and xor-4 levels inside the lane, xor 2 and xor 1 across the
        // quad): every sum formed as the 16-lane form of layer_norm_vec_kernel forms it.
        if (wave < 4) {
            const int lq = lane & 3, lrow = 16 * wave + (lane >> 2);
            const double inv_dim = 1.0 / static_cast<double>(KV);
            float4 xv[4], lnw[4], lnb[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                xv[i] = *reinterpret_cast<const float4*>(lat_f + lat_at(lrow, lq + 4 * i));
                lnw[i] = *reinterpret_cast<const float4*>(lnp_s + 4 * (lq + 4 * i));
                lnb[i] = *reinterpret_cast<const float4*>(lnp_s + KV + 4 * (lq + 4 * i));
            }
            auto row_sum = [](const double (&sg)[4]) {
                double u = (sg[0] + sg[2]) + (sg[1] + sg[3]);
                u += xor_row_d<2>(u);
                u += xor_row_d<1>(u);
                return u;
            };
            double sg[4];
#pragma unroll
            for (int i = 0; i < 4; ++i)
                sg[i] = (static_cast<double>(xv[i].x) + static_cast<double>(xv[i].y)) +
                        (static_cast<double>(xv[i].z) + static_cast<double>(xv[i].w));
            const double mean = row_sum(sg) * inv_dim;
            double ac[4][4];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                ac[i][0] = static_cast<double>(xv[i].x) - mean;
                ac[i][1] = static_cast<double>(xv[i].y) - mean;
                ac[i][2] = static_cast<double>(xv[i].z) - mean;
                ac[i][3] = static_cast<double>(xv[i].w) - mean;
                sg[i] = (ac[i][0] * ac[i][0] + ac[i][1] * ac[i][1]) + (ac[i][2] * ac[i][2] + ac[i][3] * ac[i][3]);
            }
            const double rstd = 1.0 / sqrt(fma(row_sum(sg), inv_dim, p.ln_eps));
            const uint32_t live = SPAN * t + lrow < L ? 0xffffffffu : 0u;  // keys past L: zero, as the LNIN form reads them
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const float o0 = static_cast<float>((ac[i][0] * rstd) * lnw[i].x + static_cast<double>(lnb[i].x));
                const float o1 = static_cast<float>((ac[i][1] * rstd) * lnw[i].y + static_cast<double>(lnb[i].y));
                const float o2 = static_cast<float>((ac[i][2] * rstd) * lnw[i].z + static_cast<double>(lnb[i].z));
                const float o3 = static_cast<float>((ac[i][3] * rstd) * lnw[i].w + static_cast<double>(lnb[i].w));
                *reinterpret_cast<uint2*>(lat_s + lrow * LP + 4 * (lq + 4 * i)) =
                    make_uint2(pack2(o0, o1) & live, pack2(o2, o3) & live);
            }
        }
        __syncthreads();  // the normalised latent is in LDS; the fp32 latent is dead

        // 5. kv_up of head h, column tiles 3 wg .. 3 wg + 2 over the 4 row tiles: k_nope formed transposed
        // (W_up rows as the A operand: four consecutive dims of one key per lane), v as keys x dims (four
        // consecutive keys of one dim): one 8-byte store per lane either way, the same products in the same
        // order.
        auto kv_up = [&](auto wg_c) {
            constexpr int WG = decltype(wg_c)::value;
            u16* kh = k_s + h * SPAN * HD;
            u16* vh = vt_s + h * HD * SPAN;
#pragma unroll
            for (int rt = 0; rt < RT; ++rt) {
                bf16x8 la[KV / 32];
#pragma unroll
                for (int ks = 0; ks < KV / 32; ++ks)
                    la[ks] = *reinterpret_cast<const bf16x8*>(lat_s + (16 * rt + li) * LP + 32 * ks + 8 * g);
#pragma unroll
                for (int c = 0; c < CTW; ++c) {
                    constexpr int CT0 = CTW * WG;
                    const int ct = CT0 + c;
                    f32x4 a = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
                    for (int ks = 0; ks < KV / 32; ++ks)
                        a = ct < NOPE / 16
                                ? __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, wu[c][ks]), la[ks], a, 0, 0, 0)
                                : __builtin_amdgcn_mfma_f32_16x16x32_bf16(la[ks], __builtin_bit_cast(bf16x8, wu[c][ks]), a, 0, 0, 0);
                    const uint2 e = make_uint2(pack2(a[0], a[1]), pack2(a[2], a[3]));
                    if (ct < NOPE / 16) {
                        *reinterpret_cast<uint2*>(kh + k_at(16 * rt + li, 16 * ct + 4 * g)) = e;
                    } else {
                        *reinterpret_cast<uint2*>(vh + v_at(16 * (ct - NOPE / 16) + li, 16 * rt + 4 * g)) = e;
                    }
                }
            }
        };
        if (wg == 0) {
            kv_up(std::integral_constant<int, 0>{});
        } else {
            kv_up(std::integral_constant<int, 1>{});
        }
        __syncthreads();  // k and v^T of the tile are in LDS

        // 6. The span's queries against key tile t (mla_attend_kernel's chunk t): all four 16-key tiles
        // below the diagonal tile (t < j); for t == j only the tiles at or below each query tile's
        // diagonal, the mask on the diagonal tile alone (a tile above it is all -inf in mla_attend_kernel:
        // it adds nothing to the max, +0 to the sum and zero weights to P). Keys past L lie past every
        // stored query's diagonal. The first tile starts from m = -inf, l = 0, o = 0.
        auto attend = [&](auto wg_c, auto first_c, auto diag_c) {
            constexpr int WG = decltype(wg_c)::value;
            constexpr bool FIRST = decltype(first_c)::value, DIAG = decltype(diag_c)::value;
            constexpr int QT[2] = {WG, 3 - WG};
            const u16* kh = k_s + h * SPAN * HD;
            const u16* vh = vt_s + h * HD * SPAN;
            auto unit = [&](auto i_c) {
                constexpr int I = decltype(i_c)::value;
                constexpr int NKT = DIAG ? QT[I] + 1 : 4;
                bf16x8 qb[HD / 32];
#pragma unroll
                for (int c = 0; c < HD / 32; ++c)
                    qb[c] = *reinterpret_cast<const bf16x8*>(q_s + sw(16 * QT[I] + li, HD * h + 32 * c + 8 * g));
                f32x4 sc[NKT];
#pragma unroll
                for (int kt = 0; kt < NKT; ++kt) {
                    sc[kt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
                    for (int c = 0; c < HD / 32; ++c) {
                        const bf16x8 ka = *reinterpret_cast<const bf16x8*>(kh + k_at(16 * kt + li, 32 * c + 8 * g));
                        sc[kt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ka, qb[c], sc[kt], 0, 0, 0);
                    }
                }
                float mx = -INFINITY;
#pragma unroll
                for (int kt = 0; kt < NKT; ++kt) {
#pragma unroll
                    for (int v = 0; v < 4; ++v) {
                        float xv = sc[kt][v];
                        if (DIAG && kt == QT[I]) xv = 4 * g + v <= li ? xv : -INFINITY;
                        sc[kt][v] = xv;
                        mx = fmaxf(mx, xv);
                    }
                }
                mx = fmaxf(mx, lane_xor16(mx));
                mx = fmaxf(mx, lane_xor32(mx));
                mx *= p.scale_log2;  // the max of the scaled scores (the scale is positive)
                const float m_new = FIRST ? mx : fmaxf(m_run[I], mx);
                const float m_use = m_new == -INFINITY ? 0.0f : m_new;
                float corr = 0.0f;
                if constexpr (!FIRST) corr = __builtin_amdgcn_exp2f(m_run[I] - m_use);
                m_run[I] = m_new;
                float psum = 0.0f;
#pragma unroll
                for (int kt = 0; kt < NKT; ++kt) {
#pragma unroll
                    for (int v = 0; v < 4; ++v) {
                        const float e = __builtin_amdgcn_exp2f(fmaf(sc[kt][v], p.scale_log2, -m_use));
                        sc[kt][v] = e;
                        psum += e;
                    }
                }
                if constexpr (FIRST) {
                    l_run[I] = psum;
                } else {
                    l_run[I] = l_run[I] * corr + psum;
#pragma unroll
                    for (int ot = 0; ot < HD / 16; ++ot)
#pragma unroll
                        for (int v = 0; v < 4; ++v) o[I][ot][v] *= corr;
                }
#pragma unroll
                for (int half = 0; half < 2; ++half) {
                    if (2 * half >= NKT) continue;  // P is zero over both key tiles (known at compile time)
                    const int ta = 2 * half, tb = 2 * half + 1 < NKT ? 2 * half + 1 : ta;
                    const uint2 pa = make_uint2(pack2(sc[ta][0], sc[ta][1]), pack2(sc[ta][2], sc[ta][3]));
                    const uint2 pz = 2 * half + 1 < NKT ? make_uint2(pack2(sc[tb][0], sc[tb][1]), pack2(sc[tb][2], sc[tb][3]))
                                                        : make_uint2(0u, 0u);
                    const bf16x8 pb = __builtin_bit_cast(bf16x8, uint4{pa.x, pa.y, pz.x, pz.y});
#pragma unroll
                    for (int ot = 0; ot < HD / 16; ++ot) {
                        const int dim = 16 * ot + li, key0 = 32 * half + 4 * g;
                        const uint2 lo = *reinterpret_cast<const uint2*>(vh + v_at(dim, key0));
                        const uint2 hi = *reinterpret_cast<const uint2*>(vh + v_at(dim, key0 + 16));
                        const uint4 raw = {lo.x, lo.y, hi.x, hi.y};
                        o[I][ot] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, raw), pb, o[I][ot],
                                                                            0, 0, 0);
                    }
                }
            };
            unit(std::integral_constant<int, 0>{});
            __builtin_amdgcn_sched_barrier(0);  // one unit's operands in registers at a time
            unit(std::integral_constant<int, 1>{});
        };
        using T_ = std::true_type;
        using F_ = std::false_type;
        auto attend_wg = [&](auto first_c, auto diag_c) {
            if (wg == 0) {
                attend(std::integral_constant<int, 0>{}, first_c, diag_c);
            } else {
                attend(std::integral_constant<int, 1>{}, first_c, diag_c);
            }
        };
        if (t == 0) {
            if (t == j) attend_wg(T_{}, T_{}); else attend_wg(T_{}, F_{});
        } else {
            if (t == j) attend_wg(F_{}, T_{}); else attend_wg(F_{}, F_{});
        }
    }

    // 7. Normalised output, rounded to bf16 as the o_proj takes it, into x's place (rows past L are not
    // stored by the o_proj and are left as they are); the o_proj fragments in flight meanwhile.
    uint4 wo[2][D / 32];
#pragma unroll
    for (int c = 0; c < 2; ++c)
#pragma unroll
        for (int s = 0; s < D / 32; ++s)
            wo[c][s] = *reinterpret_cast<const uint4*>(PACKED ? p.w_out + (((2 * wave + c) * (D / 32) + s) * 64 + lane) * 8
                                                              : p.w_out + (16 * (2 * wave + c) + li) * D + 32 * s + 8 * g);
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const int r = 16 * (i == 0 ? wg : 3 - wg) + li;
        float l = l_run[i] + lane_xor16(l_run[i]);
        l = l + lane_xor32(l);
        if (SPAN * j + r >= L) continue;
        const float inv = 1.0f / l;
#pragma unroll
        for (int ot = 0; ot < HD / 16; ++ot)
            *reinterpret_cast<uint2*>(x_s + sw(r, HD * h + 16 * ot + 4 * g)) =
                make_uint2(pack2(o[i][ot][0] * inv, o[i][ot][1] * inv), pack2(o[i][ot][2] * inv, o[i][ot][3] * inv));
    }
    __syncthreads();

    // 8. o_proj: wave w computes output columns 32 w .. 32 w + 31 of the span's rows, two row tiles at a
    // time (four chains, each the linear's chain over the 8 k steps).
    float* orow0 = p.out + (b * L + SPAN * j) * static_cast<int64_t>(D);
#pragma unroll
    for (int m = 0; m < RT; m += 2) {
        bf16x8 af[2][D / 32];
#pragma unroll
        for (int mm = 0; mm < 2; ++mm)
#pragma unroll
            for (int s = 0; s < D / 32; ++s)
                af[mm][s] = *reinterpret_cast<const bf16x8*>(x_s + sw(16 * (m + mm) + li, 32 * s + 8 * g));
        f32x4 y[2][2];
#pragma unroll
        for (int mm = 0; mm < 2; ++mm)
#pragma unroll
            for (int c = 0; c < 2; ++c) y[mm][c] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int s = 0; s < D / 32; ++s)
#pragma unroll
            for (int mm = 0; mm < 2; ++mm)
#pragma unroll
                for (int c = 0; c < 2; ++c)
                    y[mm][c] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, wo[c][s]), af[mm][s],
                                                                       y[mm][c], 0, 0, 0);
#pragma unroll
        for (int mm = 0; mm < 2; ++mm) {
            const int row = 16 * (m + mm) + li;
            if (SPAN * j + row < L) {
#pragma unroll
                for (int c = 0; c < 2; ++c)
                    *reinterpret_cast<f32x4*>(orow0 + row * D + 32 * wave + 16 * c + 4 * g) = y[mm][c] + f32x4{0.f, 0.f, 0.f, 0.f};
            }
        }
    }
}

// The weights of the one-launch kernels into their packed layouts (MlaPack<8>
// for mla_window_kernel<8, true>, MlaSpanPack for mla_span_kernel<true>), one
// 16-byte unit per thread (a copy: every unit is one unit of the row-major
// weight).
template <typename P>
__global__ __launch_bounds__(256) void mla_pack_kernel(const u16* w_in, const u16* w_up, const u16* w_out, u16* packed) {
    const int u = static_cast<int>(blockIdx.x) * 256 + static_cast<int>(threadIdx.x);
    if (u >= P::UNITS) return;
    const int lane = u % 64, r = lane % 16, g = lane / 16;
    constexpr int KS = P::D / 32, US = P::KV / 32;
    const u16* src;
    if (u < P::IN_UNITS) {
        const int tile = u / (KS * 64), s = (u / 64) % KS;
        src = w_in + P::in_row(tile, r) * P::D + 32 * s + 8 * g;
    } else if (u < P::IN_UNITS + P::UP_UNITS) {
        const int v = u - P::IN_UNITS;
        const int head = v / (P::CT * US * 64), ct = (v / (US * 64)) % P::CT, ks = (v / 64) % US;
        src = w_up + (head * P::UPW + 16 * ct + r) * P::KV + 32 * ks + 8 * g;
    } else {
        const int v = u - P::IN_UNITS - P::UP_UNITS;
        const int tile = v / (KS * 64), s = (v / 64) % KS;
        src = w_out + (16 * tile + r) * P::D + 32 * s + 8 * g;
    }
    reinterpret_cast<uint4*>(packed)[u] = *reinterpret_cast<const uint4*>(src);
}

}  // namespace
}  // namespace mlk

using namespace mlk;

extern "C" mlk_status mlk_mla_rope_qk(float* q, int64_t q_token_stride, int64_t q_length, const float* kv,
                                      const float* k_rope, int64_t k_rope_token_stride, const float* cosine,
                                      const float* sine, int64_t batch, int64_t length, int64_t heads,
                                      int64_t head_dim, int64_t nope_dim, float* k, mlk_stream_t stream) {
    const int64_t rope_dim = head_dim - nope_dim;
    MLK_CHECK(nope_dim >= 0 && rope_dim > 0 && rope_dim % 2 == 0, "head_dim - nope_dim must be a positive even rope_dim");
    MLK_CHECK(q_length >= 1 && q_length <= length, "q must cover between 1 and L trailing positions");
    MLK_CHECK(batch >= 0 && heads > 0, "invalid MLA geometry");
    MLK_CHECK(q_token_stride >= heads * head_dim, "q token stride must cover every head");
    MLK_CHECK(k_rope_token_stride >= rope_dim, "k_rope token stride must cover rope_dim");
    if (batch == 0) return MLK_OK;
    MLK_CHECK(q && kv && k_rope && cosine && sine && k, "null tensor pointer");
    RopeArgs p{q, q_token_stride, q_length, kv, k_rope, k_rope_token_stride, cosine, sine, k,
               batch, length, heads, head_dim, nope_dim};
    const int64_t threads = batch * length * heads * (nope_dim + rope_dim / 2);
    const dim3 grid(static_cast<unsigned>(ceil_div(threads, 256)));
    if (threads < (int64_t{1} << 31)) {
        hipLaunchKernelGGL(rope_kernel<uint32_t>, grid, dim3(256), 0, reinterpret_cast<hipStream_t>(stream), p);
    } else {
        hipLaunchKernelGGL(rope_kernel<int64_t>, grid, dim3(256), 0, reinterpret_cast<hipStream_t>(stream), p);
    }
    return launch_status("mla rope");
}

extern "C" mlk_status mlk_attention(const float* q, int64_t q_token_stride, int64_t q_head_stride, const float* k,
                                    int64_t k_token_stride, int64_t k_head_stride, const float* v,
                                    int64_t v_token_stride, int64_t v_head_stride, int64_t batch, int64_t heads,
                                    int64_t q_length, int64_t kv_length, int64_t head_dim, int32_t mask,
                                    double scale, int32_t precision, float* out, mlk_stream_t stream) {
    MLK_CHECK(batch >= 0 && heads > 0 && head_dim > 0 && q_length >= 1 && kv_length >= 1, "invalid attention geometry");
    MLK_CHECK(head_dim <= 128, "head_dim above 128 is not supported");
    MLK_CHECK(mask >= MLK_MASK_NONE && mask <= MLK_MASK_CAUSAL_BOTTOM_RIGHT, "unknown attention mask");
    MLK_CHECK(mask != MLK_MASK_CAUSAL_BOTTOM_RIGHT || q_length <= kv_length,
              "a bottom-right causal mask needs q_length <= kv_length");
    MLK_CHECK(precision == MLK_DTYPE_F32 || precision == MLK_DTYPE_BF16, "precision must be f32 or bf16");
    MLK_CHECK(batch <= 65535 && heads <= 65535, "too many windows or heads for one launch");
    if (batch == 0) return MLK_OK;
    MLK_CHECK(q && k && v && out, "null tensor pointer");
    AttnArgs p{};
    p.q = q;
    p.q_ts = q_token_stride;
    p.q_hs = q_head_stride;
    p.k = k;
    p.k_ts = k_token_stride;
    p.k_hs = k_head_stride;
    p.v = v;
    p.v_ts = v_token_stride;
    p.v_hs = v_head_stride;
    p.out = out;
    p.batch = batch;
    p.heads = heads;
    p.q_length = q_length;
    p.kv_length = kv_length;
    p.head_dim = head_dim;
    p.offset = mask == MLK_MASK_NONE ? kv_length : (mask == MLK_MASK_CAUSAL_TOP_LEFT ? 0 : kv_length - q_length);
    p.scale_log2 = static_cast<float>(scale * 1.4426950408889634);
    const bool vec = aligned16(q) && aligned16(k) && aligned16(v) && aligned16(out) && q_token_stride % 4 == 0 &&
                     q_head_stride % 4 == 0 && k_token_stride % 4 == 0 && k_head_stride % 4 == 0 &&
                     v_token_stride % 4 == 0 && v_head_stride % 4 == 0 && head_dim % 4 == 0;
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    if (precision == MLK_DTYPE_BF16) {
        dispatch_attn<true>(p, vec, s);
    } else {
        dispatch_attn<false>(p, vec, s);
    }
    return launch_status("attention");
}

extern "C" mlk_status mlk_mla_attend(const float* projected, int64_t batch, int64_t length, int64_t proj_token_stride,
                                     int64_t q_offset, int64_t kv_offset, int64_t k_rope_offset, int64_t heads,
                                     int64_t head_dim, int64_t nope_dim, int64_t kv_rank, const float* kv_norm_w,
                                     const float* kv_norm_b, double kv_norm_eps, const void* kv_up_weight,
                                     const float* cosine, const float* sine, double scale, float* out,
                                     mlk_stream_t stream) {
    MLK_CHECK(batch >= 0 && length >= 1 && heads > 0, "invalid MLA geometry");
    const bool cfg32 = head_dim == 32 && nope_dim == 16 && kv_rank == 64 && length <= 128;
    const bool cfg64 = head_dim == 64 && nope_dim == 32 && kv_rank == 64 && length <= 256;
    if (!cfg32 && !cfg64) {
        set_error("mla_attend: geometry without a fused kernel (use the separate operators)");
        return MLK_ERR_UNSUPPORTED;
    }
    if (k_rope_offset % 4 != 0 || !aligned16(cosine) || !aligned16(sine)) {
        set_error("mla_attend: k_rope and the cos/sin tables are read as 16-byte vectors (use the separate operators)");
        return MLK_ERR_UNSUPPORTED;
    }
    MLK_CHECK(proj_token_stride % 4 == 0 && q_offset % 4 == 0 && kv_offset % 4 == 0 && aligned16(projected) &&
                  aligned16(kv_norm_w) && (kv_norm_b == nullptr || aligned16(kv_norm_b)) && aligned16(kv_up_weight) &&
                  aligned16(out),
              "mla_attend: operands must be 16-byte aligned");
    if (batch == 0) return MLK_OK;
    MLK_CHECK(projected && kv_norm_w && kv_up_weight && cosine && sine && out, "null tensor pointer");
    MLK_CHECK(batch * heads <= 0x7fffffff, "too many windows x heads for one launch");
    MlaAttendArgs p{projected, proj_token_stride, q_offset, kv_offset, k_rope_offset, kv_norm_w, kv_norm_b,
                    static_cast<double>(static_cast<float>(kv_norm_eps)), static_cast<const u16*>(kv_up_weight),
                    cosine, sine, out, batch, heads, length, static_cast<float>(scale * 1.4426950408889634)};
    const dim3 grid(static_cast<unsigned>(batch * heads));
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    if (cfg32) {
        if (p.scale_log2 > 0.0f) {
            hipLaunchKernelGGL((mla_attend_kernel<32, 16, 64, 4, 2, false, true>), grid, dim3(256), 0, s, p);
        } else {
            hipLaunchKernelGGL((mla_attend_kernel<32, 16, 64, 4, 2, false, false>), grid, dim3(256), 0, s, p);
        }
    } else {
        if (p.scale_log2 > 0.0f) {
            hipLaunchKernelGGL((mla_attend_kernel<64, 32, 64, 8, 2, false, true>), grid, dim3(512), 0, s, p);
        } else {
            hipLaunchKernelGGL((mla_attend_kernel<64, 32, 64, 8, 2, false, false>), grid, dim3(512), 0, s, p);
        }
    }
    return launch_status("mla_attend");
}

extern "C" mlk_status mlk_mla_attend_normed(const float* projected, int64_t batch, int64_t length,
                                            int64_t proj_token_stride, int64_t q_offset, int64_t k_rope_offset,
                                            int64_t heads, int64_t head_dim, int64_t nope_dim, int64_t kv_rank,
                                            const void* latent_normed, const void* kv_up_weight,
                                            const float* cosine, const float* sine, double scale, float* out,
                                            mlk_stream_t stream) {
    MLK_CHECK(batch >= 0 && length >= 1 && heads > 0, "invalid MLA geometry");
    const bool cfg32 = head_dim == 32 && nope_dim == 16 && kv_rank == 64 && length <= 128;
    const bool cfg64 = head_dim == 64 && nope_dim == 32 && kv_rank == 64 && length <= 256;
    if (!cfg32 && !cfg64) {
        set_error("mla_attend: geometry without a fused kernel (use the separate operators)");
        return MLK_ERR_UNSUPPORTED;
    }
    if (k_rope_offset % 4 != 0 || !aligned16(cosine) || !aligned16(sine)) {
        set_error("mla_attend: k_rope and the cos/sin tables are read as 16-byte vectors (use the separate operators)");
        return MLK_ERR_UNSUPPORTED;
    }
    MLK_CHECK(proj_token_stride % 4 == 0 && q_offset % 4 == 0 && aligned16(projected) && aligned16(latent_normed) &&
                  aligned16(kv_up_weight) && aligned16(out),
              "mla_attend: operands must be 16-byte aligned");
    if (batch == 0) return MLK_OK;
    MLK_CHECK(projected && latent_normed && kv_up_weight && cosine && sine && out, "null tensor pointer");
    MLK_CHECK(batch * heads <= 0x7fffffff, "too many windows x heads for one launch");
    MlaAttendArgs p{projected, proj_token_stride, q_offset, 0, k_rope_offset, nullptr, nullptr, 0.0,
                    static_cast<const u16*>(kv_up_weight), cosine, sine, out, batch, heads, length,
                    static_cast<float>(scale * 1.4426950408889634), static_cast<const u16*>(latent_normed)};
    const dim3 grid(static_cast<unsigned>(batch * heads));
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    if (cfg32) {
        if (p.scale_log2 > 0.0f) {
            hipLaunchKernelGGL((mla_attend_kernel<32, 16, 64, 4, 2, true, true>), grid, dim3(256), 0, s, p);
        } else {
            hipLaunchKernelGGL((mla_attend_kernel<32, 16, 64, 4, 2, true, false>), grid, dim3(256), 0, s, p);
        }
    } else {
        if (p.scale_log2 > 0.0f) {
            hipLaunchKernelGGL((mla_attend_kernel<64, 32, 64, 8, 2, true, true>), grid, dim3(512), 0, s, p);
        } else {
            hipLaunchKernelGGL((mla_attend_kernel<64, 32, 64, 8, 2, true, false>), grid, dim3(512), 0, s, p);
        }
    }
    return launch_status("mla_attend_normed");
}

namespace {

// The geometries the one-launch kernels are built for (mla_window_kernel: 8 heads of 32, L <= 128;
// mla_span_kernel: 4 heads of 64, L <= 256), and their operand checks; MLK_OK when a kernel takes the
// call, MLK_ERR_UNSUPPORTED (with the reason) when the separate operators must run it.
mlk_status mla_window_supported(const float* x, int64_t length, int64_t d_model, int64_t x_batch_stride,
                                int64_t x_token_stride, const float* kv_norm_w, const float* kv_norm_b,
                                const float* cosine, const float* sine, int64_t heads, int64_t head_dim,
                                int64_t nope_dim, int64_t kv_rank, double scale, const float* out,
                                std::initializer_list<const void*> weights) {
    const bool window = heads == 8 && head_dim == 32 && nope_dim == 16 && kv_rank == 64 && length <= 128;
    const bool span = heads == 4 && head_dim == 64 && nope_dim == 32 && kv_rank == 64 && length <= 256;
    if (!(window || span) || d_model != heads * head_dim) {
        set_error("mla_forward: geometry without a one-launch kernel (use the separate operators)");
        return MLK_ERR_UNSUPPORTED;
    }
    if (!(static_cast<float>(scale * 1.4426950408889634) > 0.0f)) {
        set_error("mla_forward: the per-window kernel takes a positive softmax scale (use the separate operators)");
        return MLK_ERR_UNSUPPORTED;
    }
    bool aligned = aligned16(x) && x_token_stride % 4 == 0 && x_batch_stride % 4 == 0 && aligned16(cosine) &&
                   aligned16(sine) && aligned16(kv_norm_w) && (kv_norm_b == nullptr || aligned16(kv_norm_b)) &&
                   aligned16(out);
    for (const void* w : weights) aligned = aligned && aligned16(w);
    if (!aligned) {
        set_error("mla_forward: operands must be 16-byte aligned for the per-window kernel (use the separate operators)");
        return MLK_ERR_UNSUPPORTED;
    }
    return MLK_OK;
}

mlk_status mla_window_launch(const float* x, int64_t batch, int64_t length, int64_t d_model, int64_t x_batch_stride,
                             int64_t x_token_stride, const void* w_in, const float* kv_norm_w, const float* kv_norm_b,
                             double kv_norm_eps, const void* w_up, const void* w_out, const float* cosine,
                             const float* sine, double scale, float* out, int64_t heads, bool packed,
                             mlk_stream_t stream) {
    MLK_CHECK(x_token_stride >= d_model && (length == 1 || x_batch_stride >= length * x_token_stride),
              "x strides must cover the rows");
    if (batch == 0) return MLK_OK;
    MLK_CHECK(x && w_in && kv_norm_w && w_up && w_out && cosine && sine && out, "null tensor pointer");
    MLK_CHECK(batch <= 0x7fffffff, "too many windows for one launch");
    MlaWindowArgs p{x, x_batch_stride, x_token_stride, static_cast<const u16*>(w_in), kv_norm_w, kv_norm_b,
                    static_cast<double>(static_cast<float>(kv_norm_eps)), static_cast<const u16*>(w_up),
                    static_cast<const u16*>(w_out), cosine, sine, out, length,
                    static_cast<float>(scale * 1.4426950408889634)};
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    if (heads == 4) {  // mla_span_kernel: one block per (window, 64 query rows)
        const int64_t spans = (length + 63) / 64;
        MLK_CHECK(batch * spans <= 0x7fffffff, "too many windows for one launch");
        const dim3 grid(static_cast<unsigned>(batch * spans));
        if (packed) {
            hipLaunchKernelGGL((mla_span_kernel<true>), grid, dim3(512), 0, s, p, static_cast<int>(spans));
        } else {
            hipLaunchKernelGGL((mla_span_kernel<false>), grid, dim3(512), 0, s, p, static_cast<int>(spans));
        }
        return launch_status("mla_forward");
    }
    const dim3 grid(static_cast<unsigned>(batch));
    if (packed) {
        hipLaunchKernelGGL((mla_window_kernel<8, true>), grid, dim3(512), 0, s, p);
    } else {
        hipLaunchKernelGGL((mla_window_kernel<8, false>), grid, dim3(512), 0, s, p);
    }
    return launch_status("mla_forward");
}

}  // namespace

extern "C" mlk_status mlk_mla_forward(const float* x, int64_t batch, int64_t length, int64_t d_model,
                                      int64_t x_batch_stride, int64_t x_token_stride, const void* in_proj_weight,
                                      const float* kv_norm_w, const float* kv_norm_b, double kv_norm_eps,
                                      const void* kv_up_weight, const void* out_weight, const float* cosine,
                                      const float* sine, int64_t heads, int64_t head_dim, int64_t nope_dim,
                                      int64_t kv_rank, int32_t weight_dtype, double scale, float* out,
                                      mlk_stream_t stream) {
    MLK_CHECK(batch >= 0 && length >= 1 && heads > 0 && d_model == heads * head_dim, "invalid MLA geometry");
    if (weight_dtype != MLK_DTYPE_BF16) {
        set_error("mla_forward: the per-window kernel takes bf16 weights (use the separate operators)");
        return MLK_ERR_UNSUPPORTED;
    }
    const mlk_status ok = mla_window_supported(x, length, d_model, x_batch_stride, x_token_stride, kv_norm_w, kv_norm_b,
                                               cosine, sine, heads, head_dim, nope_dim, kv_rank, scale, out,
                                               {in_proj_weight, kv_up_weight, out_weight});
    if (ok != MLK_OK) return ok;
    return mla_window_launch(x, batch, length, d_model, x_batch_stride, x_token_stride, in_proj_weight, kv_norm_w,
                             kv_norm_b, kv_norm_eps, kv_up_weight, out_weight, cosine, sine, scale, out, heads, false,
                             stream);
}

extern "C" int64_t mlk_mla_packed_elems(int64_t d_model, int64_t heads, int64_t head_dim, int64_t nope_dim,
                                        int64_t kv_rank) {
    if (d_model != heads * head_dim || kv_rank != 64) return 0;
    if (heads == 8 && head_dim == 32 && nope_dim == 16) return static_cast<int64_t>(MlaPack<8>::UNITS) * 8;
    if (heads == 4 && head_dim == 64 && nope_dim == 32) return static_cast<int64_t>(MlaSpanPack::UNITS) * 8;
    return 0;
}

extern "C" mlk_status mlk_mla_pack_weights(const void* in_proj_weight, const void* kv_up_weight, const void* out_weight,
                                           int64_t d_model, int64_t heads, int64_t head_dim, int64_t nope_dim,
                                           int64_t kv_rank, int32_t weight_dtype, void* packed, mlk_stream_t stream) {
    if (weight_dtype != MLK_DTYPE_BF16 || mlk_mla_packed_elems(d_model, heads, head_dim, nope_dim, kv_rank) == 0) {
        set_error("mla_pack_weights: geometry without a one-launch kernel (bf16; 8 heads of 32, rope 16, or 4 heads of 64, "
                  "rope 32; kv rank 64)");
        return MLK_ERR_UNSUPPORTED;
    }
    MLK_CHECK(in_proj_weight && kv_up_weight && out_weight && packed, "null tensor pointer");
    MLK_CHECK(aligned16(in_proj_weight) && aligned16(kv_up_weight) && aligned16(out_weight) && aligned16(packed),
              "mla_pack_weights: operands must be 16-byte aligned");
    const bool span = heads == 4;
    const int units = span ? MlaSpanPack::UNITS : MlaPack<8>::UNITS;
    const dim3 grid(static_cast<unsigned>((units + 255) / 256));
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    const u16* wi = static_cast<const u16*>(in_proj_weight);
    const u16* wu = static_cast<const u16*>(kv_up_weight);
    const u16* wo = static_cast<const u16*>(out_weight);
    if (span) {
        hipLaunchKernelGGL((mla_pack_kernel<MlaSpanPack>), grid, dim3(256), 0, s, wi, wu, wo, static_cast<u16*>(packed));
    } else {
        hipLaunchKernelGGL((mla_pack_kernel<MlaPack<8>>), grid, dim3(256), 0, s, wi, wu, wo, static_cast<u16*>(packed));
    }
    return launch_status("mla_pack_weights");
}

extern "C" mlk_status mlk_mla_forward_packed(const float* x, int64_t batch, int64_t length, int64_t d_model,
                                             int64_t x_batch_stride, int64_t x_token_stride, const void* packed_weights,
                                             const float* kv_norm_w, const float* kv_norm_b, double kv_norm_eps,
                                             const float* cosine, const float* sine, int64_t heads, int64_t head_dim,
                                             int64_t nope_dim, int64_t kv_rank, double scale, float* out,
                                             mlk_stream_t stream) {
    MLK_CHECK(batch >= 0 && length >= 1 && heads > 0 && d_model == heads * head_dim, "invalid MLA geometry");
    if (mlk_mla_packed_elems(d_model, heads, head_dim, nope_dim, kv_rank) == 0) {
        set_error("mla_forward_packed: geometry without packed weights (8 heads of 32, rope 16, or 4 heads of 64, rope 32; "
                  "kv rank 64)");
        return MLK_ERR_UNSUPPORTED;
    }
    const mlk_status ok = mla_window_supported(x, length, d_model, x_batch_stride, x_token_stride, kv_norm_w, kv_norm_b,
                                               cosine, sine, heads, head_dim, nope_dim, kv_rank, scale, out,
                                               {packed_weights});
    if (ok != MLK_OK) return ok;
    const u16* w = static_cast<const u16*>(packed_weights);
    const int64_t in_units = heads == 4 ? MlaSpanPack::IN_UNITS : MlaPack<8>::IN_UNITS;
    const int64_t up_units = heads == 4 ? MlaSpanPack::UP_UNITS : MlaPack<8>::UP_UNITS;
    return mla_window_launch(x, batch, length, d_model, x_batch_stride, x_token_stride, w, kv_norm_w, kv_norm_b,
                             kv_norm_eps, w + 8 * in_units, w + 8 * (in_units + up_units), cosine, sine, scale, out,
                             heads, true, stream);
}
