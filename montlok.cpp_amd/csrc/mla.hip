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
// transposed in LDS. Running max, running sum and rescale are per lane.
//   BF16: v_mfma_f32_16x16x32_bf16, q/k/v and p rounded to bf16, fp32
//         accumulation and fp32 softmax (bf16-weight configurations).
//   FP32: v_mfma_f32_16x16x4_f32, fp32 throughout (fp32 configurations).

#include "mlk_common.h"

namespace mlk {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
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

template <int HD, bool BF16, bool VEC>
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
                    const float x = ok ? s[t][v] * p.scale_log2 : -INFINITY;
                    s[t][v] = x;
                    mx = fmaxf(mx, x);
                }
            }
            mx = xor_max(mx, 16);
            mx = xor_max(mx, 32);
            const float m_new = fmaxf(m_run[i], mx);
            const float m_use = m_new == -INFINITY ? 0.0f : m_new;
            const float corr = __builtin_amdgcn_exp2f(m_run[i] - m_use);
            m_run[i] = m_new;
            float psum = 0.0f;
#pragma unroll
            for (int t = 0; t < 4; ++t) {
#pragma unroll
                for (int v = 0; v < 4; ++v) {
                    const float e = __builtin_amdgcn_exp2f(s[t][v] - m_use);
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
    if (vec) {
        hipLaunchKernelGGL((attn_kernel<HD, BF16, true>), grid, dim3(256), 0, stream, p);
    } else {
        hipLaunchKernelGGL((attn_kernel<HD, BF16, false>), grid, dim3(256), 0, stream, p);
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
