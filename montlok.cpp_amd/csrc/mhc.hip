// Manifold-constrained hyper-connection (mHC) residual mix on gfx950.
//
// Read side (mhc_prepare, reference rdt4quant_cpu/montlok_mhc.h:198-322), per
// token of n streams x d:
//   ref    = RMSNorm_d(mean_i streams_i) * norm_w          (double)
//   logits = tanh(W64 . ref), W64 = cat(pre, post, res projections) [2n+n^2, d]
//   pre    = sigmoid(pre_b + a_pre * logit)                 -> fp32
//   post   = 2 * sigmoid(post_b + a_post * logit)           -> fp32
//   res    = Sinkhorn(exp(res_b + a_res * logit)), max(iters, 1) rounds of row
//            then column normalisation in double            -> fp32
//   agg    = sum_i double(pre_i) * streams_i (one rounding), optionally
//            RMSNorm'd in place with agg_norm_w.
// Write side (mhc_combine, montlok_mhc.h:336-438):
//   new_i = double(post_i) * out + sum_j double(res_ij) * streams_j (one
//   rounding), collapsed = mean_i of the rounded new_i (double, one rounding).
//
// Kernels
//   prepare_n4<D> (n = 4, d = D in {64, 128, 256, 512}): one 256-thread block
//     per 16 tokens. In the load and MFMA phase lane l of every wave is
//     (token t = l % 16, k-lane q = l / 16). The 24 dot products of each token
//     run on the fp64 matrix cores, v_mfma_f64_16x16x4_f64: A = 16 projection
//     rows x 4 k, B = 4 k x 16 tokens, two row tiles (tile 0 = the 16 res rows,
//     tile 1 = 4 pre + 4 post rows + 8 zero rows). The k range is split over
//     the block's four waves (wave w owns k in [w*D/4, (w+1)*D/4)); partial
//     tiles go through LDS and are summed in wave order. norm_w and the RMS
//     scale are applied on the B side and after the sum:
//     logit = scale * sum_k W[r,k] * (w_k * m_k). In the coefficient phase
//     each wave takes 4 tokens with one res entry per lane (token 4w + l / 16,
//     entry l % 16; lanes with entry < 8 also produce pre or post). Sinkhorn
//     row sums are quad sums and column sums 16-lane sums (DPP, the
//     reference's association), the reciprocals the IEEE quotient 1 / s.
//     Traffic per token: n*d*4 bytes read once + d*4 written + 36 floats of
//     coefficients (non-temporal stores).
//   prepare_generic: one wave per token, every sum in the reference's own
//     order (bit-exact with it); used for other n or d. Slow, small shapes.
//   combine<N>: one thread per (token, float4 of d), or per (token, two
//     float4 d / 2 apart) for n = 4 with the new streams written, HBM-bound.
#include "mlk_common.h"

namespace mlk {
namespace {

typedef float nt_f4 __attribute__((ext_vector_type(4)));  // for non-temporal vector loads and stores

typedef double double4_t __attribute__((ext_vector_type(4)));

constexpr int kBlock = 256;

__device__ __forceinline__ double sigmoid_d(double x) { return 1.0 / (1.0 + exp(-x)); }

// DPP moves of a double (two 32-bit halves). Control words (GFX9 DPP):
// quad_perm [1,0,3,2] = 0xB1, quad_perm [2,3,0,1] = 0x4E, row_ror:4 = 0x124,
// row_ror:8 = 0x128.
template <int CTRL>
__device__ __forceinline__ double dpp_d(double v) {
    const int lo = __builtin_amdgcn_mov_dpp(__double2loint(v), CTRL, 0xF, 0xF, false);
    const int hi = __builtin_amdgcn_mov_dpp(__double2hiint(v), CTRL, 0xF, 0xF, false);
    return __hiloint2double(hi, lo);
}

// Sum over the 4 lanes of a quad (a row of a 4x4 matrix held one entry per
// lane, entry e = 4i + j at lane e of a 16-lane group): (x0 + x1) + (x2 + x3)
// by commutativity bit-identical in all four lanes.
__device__ __forceinline__ double quad_sum(double v) {
    const double s = v + dpp_d<0xB1>(v);
    return s + dpp_d<0x4E>(s);
}

// Sum over lanes j, j+4, j+8, j+12 of a 16-lane group (a column of the
// matrix): (m[i] + m[i+2]) + (m[i+1] + m[i+3]), identical in all four rows.
__device__ __forceinline__ double column_sum(double v) {
    const double s = v + dpp_d<0x128>(v);
    return s + dpp_d<0x124>(s);
}

// ---------------------------------------------------------------------------
// prepare, n = 4 fast path
// ---------------------------------------------------------------------------

struct PrepareArgs {
    const float* streams;
    int64_t tokens;
    int64_t sd;  // stream stride (0: broadcast backbone)
    int64_t ts;  // token stride
    const float* norm_w;
    double eps;
    const double* proj_w;  // [24, D]: pre rows 0-3, post rows 4-7, res rows 8-23
    const float* pre_bias;
    const float* post_bias;
    const float* res_bias;
    const float* pre_alpha;
    const float* post_alpha;
    const float* res_alpha;
    int iters;
    const float* agg_norm_w;
    double agg_norm_eps;
    float* agg;
    float* pre;
    float* post;
    float* res;
    // Fused write of the previous residual (mhc_combine_prepare): its res
    // [T, 16] and post [T, 4] coefficients, the mixer output [T, D], and the
    // new streams [T, 4, D] written on the way.
    const float* c_res;
    const float* c_post;
    const float* c_out;
    float* c_new;
};

// Values held by lanes (t, 0..3) of a wave, gathered into every lane of
// token t with the gfx950 cross-row swaps: permlane16_swap pairs rows
// (0,1) and (2,3), permlane32_swap then pairs the halves. Three VALU
// operations per dword, no LDS traffic.
__device__ __forceinline__ void gather_rows(double v, double x[4]) {
    const int lo = __double2loint(v);
    const int hi = __double2hiint(v);
    const auto p_lo = __builtin_amdgcn_permlane16_swap(lo, lo, false, false);  // {r0 r0 r2 r2}, {r1 r1 r3 r3}
    const auto p_hi = __builtin_amdgcn_permlane16_swap(hi, hi, false, false);
    const auto e_lo = __builtin_amdgcn_permlane32_swap(p_lo[0], p_lo[0], false, false);  // {r0}, {r2}
    const auto e_hi = __builtin_amdgcn_permlane32_swap(p_hi[0], p_hi[0], false, false);
    const auto o_lo = __builtin_amdgcn_permlane32_swap(p_lo[1], p_lo[1], false, false);  // {r1}, {r3}
    const auto o_hi = __builtin_amdgcn_permlane32_swap(p_hi[1], p_hi[1], false, false);
    x[0] = __hiloint2double(e_hi[0], e_lo[0]);
    x[1] = __hiloint2double(o_hi[0], o_lo[0]);
    x[2] = __hiloint2double(e_hi[1], e_lo[1]);
    x[3] = __hiloint2double(o_hi[1], o_lo[1]);
}

// The value of lane (t, 0) in every lane (t, q).
__device__ __forceinline__ float bcast_row0(float v) {
    const int bits = __float_as_int(v);
    const auto p = __builtin_amdgcn_permlane16_swap(bits, bits, false, false);
    const auto e = __builtin_amdgcn_permlane32_swap(p[0], p[0], false, false);
    return __int_as_float(e[0]);
}

// Output stores: non-temporal (NTS), or plain, where L2 merges the 64-byte
// pieces of the token rows into whole lines before they go to HBM (the large
// fused combine + prepare; the host picks).
template <bool NTS>
__device__ __forceinline__ void store_f4(float* dst, float4 v) {
    if constexpr (NTS) {
        __builtin_nontemporal_store(nt_f4{v.x, v.y, v.z, v.w}, reinterpret_cast<nt_f4*>(dst));
    } else {
        *reinterpret_cast<float4*>(dst) = v;
    }
}
template <bool NTS>
__device__ __forceinline__ void store_f(float* dst, float v) {
    if constexpr (NTS) {
        __builtin_nontemporal_store(v, dst);
    } else {
        *dst = v;
    }
}

// BC: the streams are a broadcast backbone (stream stride 0). The four
// stream values of a lane are then one load (the same operations follow on
// the same values, so the result is the general form's bit for bit), and the
// partial tiles reuse the projection block's LDS after a barrier, so that at
// d = 256 three blocks fit a CU (registers and LDS) instead of two.
template <int D, bool FUSED, bool NTS, bool BC = false>
__global__ __launch_bounds__(kBlock) __attribute__((amdgpu_waves_per_eu(BC ? 3 : 1)))
void mhc_prepare_n4_kernel(PrepareArgs a) {
    constexpr int n = 4;
    constexpr int GW = D / 64;  // groups of 16 k per wave; group g covers k in [16g, 16g + 16)
    static_assert(!(BC && FUSED), "the fused combine reads full streams");
    __shared__ __attribute__((aligned(16))) double w_lds[(2 * n + n * n) * (D + 2)];
    static_assert(!BC || 4 * 2 * 4 * 64 <= (2 * n + n * n) * (D + 2), "partial tiles inside the projection block");
    __shared__ double part_own[BC ? 1 : 4 * 2 * 4 * 64];
    double (*part)[2][4][64] = reinterpret_cast<double (*)[2][4][64]>(BC ? w_lds : part_own);
    __shared__ double part_sq[4][64];
    __shared__ double agg_sq_own[BC ? 1 : 4 * 64];
    double (*agg_sq)[64] = reinterpret_cast<double (*)[64]>(BC ? &part_sq[0][0] : agg_sq_own);  // BC: after part_sq's reads
    __shared__ float pre_lds[16][4];

    const int wave = threadIdx.x / kWave;
    const int l = threadIdx.x % kWave;
    const int t = l % 16;
    const int q = l / 16;
    const int64_t token = static_cast<int64_t>(blockIdx.x) * 16 + t;
    const bool valid = token < a.tokens;
    const float* base = a.streams + (valid ? token : 0) * a.ts;
    const double inv_n = 1.0 / n;

    // The projection block is staged in LDS once per block with coalesced
    // 16-byte loads (per-lane gathers of it from L2 cost as many cache lines
    // as the streams themselves). Its loads go out first, into registers, so
    // the LDS stores wait for them alone; then every other operand is fetched,
    // so the block waits for one round of loads. All loop bounds are compile
    // time: each load is issued without waiting for the one before.
    constexpr int WP = D + 2;  // row pitch in doubles: consecutive rows start 4 banks apart
    constexpr int kWPairs = (2 * n + n * n) * (D / 2);
    static_assert(kWPairs % kBlock == 0, "projection block must split evenly over the block");
    constexpr int kWPer = kWPairs / kBlock;
    double2 wreg[kWPer];
#pragma unroll
    for (int c = 0; c < kWPer; ++c) {
        const int u = threadIdx.x + c * kBlock;
        wreg[c] = *reinterpret_cast<const double2*>(a.proj_w + 2 * u);  // row u / (D/2), column 2 (u % (D/2))
    }
    // MFMA step s = 4g + r multiplies k = 16g + 4q + r: lane (t, q) owns the
    // float4 at 16g + 4q of every group g of its wave. Lanes of tokens past
    // the end read token 0 (in bounds): an MFMA column and every lane
    // reduction below stay within one token, and those tokens' results are
    // never stored.
    float4 sv[GW][n];
#pragma unroll
    for (int j = 0; j < GW; ++j) {
        const int k0 = 16 * (wave * GW + j) + 4 * q;
        if constexpr (BC) {
            sv[j][0] = *reinterpret_cast<const float4*>(base + k0);
#pragma unroll
            for (int i = 1; i < n; ++i) sv[j][i] = sv[j][0];
        } else {
#pragma unroll
            for (int i = 0; i < n; ++i) sv[j][i] = *reinterpret_cast<const float4*>(base + i * a.sd + k0);
        }
    }
    if constexpr (FUSED) {
        // The previous residual's write on this lane's k-slice of all n
        // streams, in mhc_combine's arithmetic (post_i * out + sum_j res_ij *
        // s_j in double, one rounding): the new streams are stored once and
        // are the streams this prepare reads.
        const int64_t tok = valid ? token : 0;
        const float4 r0 = reinterpret_cast<const float4*>(a.c_res + tok * 16)[0];
        const float4 r1 = reinterpret_cast<const float4*>(a.c_res + tok * 16)[1];
        const float4 r2 = reinterpret_cast<const float4*>(a.c_res + tok * 16)[2];
        const float4 r3 = reinterpret_cast<const float4*>(a.c_res + tok * 16)[3];
        const float4 pv = *reinterpret_cast<const float4*>(a.c_post + tok * 4);
        float4 ov[GW];
#pragma unroll
        for (int j = 0; j < GW; ++j) ov[j] = *reinterpret_cast<const float4*>(a.c_out + tok * D + 16 * (wave * GW + j) + 4 * q);
        // new_i = post_i * out + res_i0 s_0 + res_i1 s_1 + res_i2 s_2 + res_i3 s_3 (double, this order, one rounding)
        auto mix = [](float p, float4 r, float o, float s0, float s1, float s2, float s3) -> float {
            double acc = static_cast<double>(p) * static_cast<double>(o);
            acc = fma(static_cast<double>(r.x), static_cast<double>(s0), acc);
            acc = fma(static_cast<double>(r.y), static_cast<double>(s1), acc);
            acc = fma(static_cast<double>(r.z), static_cast<double>(s2), acc);
            acc = fma(static_cast<double>(r.w), static_cast<double>(s3), acc);
            return static_cast<float>(acc);
        };
#pragma unroll
        for (int j = 0; j < GW; ++j) {
            const float4 s0 = sv[j][0], s1 = sv[j][1], s2 = sv[j][2], s3 = sv[j][3], o = ov[j];
            const float4 n0 = make_float4(mix(pv.x, r0, o.x, s0.x, s1.x, s2.x, s3.x), mix(pv.x, r0, o.y, s0.y, s1.y, s2.y, s3.y),
                                          mix(pv.x, r0, o.z, s0.z, s1.z, s2.z, s3.z), mix(pv.x, r0, o.w, s0.w, s1.w, s2.w, s3.w));
            const float4 n1 = make_float4(mix(pv.y, r1, o.x, s0.x, s1.x, s2.x, s3.x), mix(pv.y, r1, o.y, s0.y, s1.y, s2.y, s3.y),
                                          mix(pv.y, r1, o.z, s0.z, s1.z, s2.z, s3.z), mix(pv.y, r1, o.w, s0.w, s1.w, s2.w, s3.w));
            const float4 n2 = make_float4(mix(pv.z, r2, o.x, s0.x, s1.x, s2.x, s3.x), mix(pv.z, r2, o.y, s0.y, s1.y, s2.y, s3.y),
                                          mix(pv.z, r2, o.z, s0.z, s1.z, s2.z, s3.z), mix(pv.z, r2, o.w, s0.w, s1.w, s2.w, s3.w));
            const float4 n3 = make_float4(mix(pv.w, r3, o.x, s0.x, s1.x, s2.x, s3.x), mix(pv.w, r3, o.y, s0.y, s1.y, s2.y, s3.y),
                                          mix(pv.w, r3, o.z, s0.z, s1.z, s2.z, s3.z), mix(pv.w, r3, o.w, s0.w, s1.w, s2.w, s3.w));
            sv[j][0] = n0;
            sv[j][1] = n1;
            sv[j][2] = n2;
            sv[j][3] = n3;
        }
    }
    float4 nw[GW];
#pragma unroll
    for (int j = 0; j < GW; ++j) nw[j] = *reinterpret_cast<const float4*>(a.norm_w + 16 * (wave * GW + j) + 4 * q);
    // agg_norm_w is read unconditionally (norm_w stands in when absent) so
    // that no branch separates these loads from the others.
    const float* anw_src = a.agg_norm_w != nullptr ? a.agg_norm_w : a.norm_w;
    float4 anw[GW];
#pragma unroll
    for (int j = 0; j < GW; ++j) anw[j] = *reinterpret_cast<const float4*>(anw_src + 16 * (wave * GW + j) + 4 * q);
#pragma unroll
    for (int c = 0; c < kWPer; ++c) {
        const int u = threadIdx.x + c * kBlock;
        *reinterpret_cast<double2*>(w_lds + (u / (D / 2)) * WP + 2 * (u % (D / 2))) = wreg[c];
    }
    // A operand: projection row for tile row i = l % 16. The accumulator of
    // the 16x16x4 f64 MFMA puts tile rows q, q+4, q+8, q+12 of token t in
    // lane (t, q), so tile 0 row i carries res entry (i % 4, i / 4) and lane q
    // ends with res row q; tile 1 row i carries pre[i / 4] (i % 4 == 0) or
    // post[i / 4] (i % 4 == 1), zero rows otherwise.
    const double* w_res = w_lds + (2 * n + 4 * (t % 4) + t / 4) * WP;
    const bool pp_row = t % 4 < 2;
    const double* w_pp = w_lds + ((t % 4 == 0 ? 0 : n) + t / 4) * WP;
    const int e_pre = l % 16;  // this lane's matrix entry in the coefficient phase
    const float res_bias_e = a.res_bias[e_pre];
    const float res_alpha = *a.res_alpha;
    const float pp_alpha = e_pre < 4 ? *a.pre_alpha : *a.post_alpha;
    const float pp_bias = e_pre < 4 ? a.pre_bias[e_pre % 4] : a.post_bias[e_pre % 4];
    __syncthreads();  // w_lds filled
    if constexpr (FUSED) {
        // The new streams, stored here rather than where they are computed so
        // that no register of the staging above stays live across the branch.
        if (valid) {
#pragma unroll
            for (int j = 0; j < GW; ++j) {
                float* dst = a.c_new + token * n * D + 16 * (wave * GW + j) + 4 * q;
#pragma unroll
                for (int i = 0; i < n; ++i) {
                    store_f4<NTS>(dst + i * D, sv[j][i]);
                }
            }
        }
    }
    double sq = 0.0;
    double4_t acc0 = {0.0, 0.0, 0.0, 0.0};
    double4_t acc1 = {0.0, 0.0, 0.0, 0.0};
#pragma unroll
    for (int j = 0; j < GW; ++j) {
        const int k0 = 16 * (wave * GW + j) + 4 * q;
        const float wk[4] = {nw[j].x, nw[j].y, nw[j].z, nw[j].w};
        const float s0[4] = {sv[j][0].x, sv[j][0].y, sv[j][0].z, sv[j][0].w};
        const float s1[4] = {sv[j][1].x, sv[j][1].y, sv[j][1].z, sv[j][1].w};
        const float s2[4] = {sv[j][2].x, sv[j][2].y, sv[j][2].z, sv[j][2].w};
        const float s3[4] = {sv[j][3].x, sv[j][3].y, sv[j][3].z, sv[j][3].w};
        // This group's A operands, read up front as 16-byte pairs (rows and
        // k0 are 16-byte aligned in LDS).
        const double2 r01 = *reinterpret_cast<const double2*>(w_res + k0);
        const double2 r23 = *reinterpret_cast<const double2*>(w_res + k0 + 2);
        const double2 p01 = *reinterpret_cast<const double2*>(w_pp + k0);
        const double2 p23 = *reinterpret_cast<const double2*>(w_pp + k0 + 2);
        const double wr[4] = {r01.x, r01.y, r23.x, r23.y};
        const double wp[4] = {pp_row ? p01.x : 0.0, pp_row ? p01.y : 0.0, pp_row ? p23.x : 0.0, pp_row ? p23.y : 0.0};
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            // m = ((s0 + s1) + s2) + s3, then * (1/n): the reference's order.
            double m = static_cast<double>(s0[r]);
            m += static_cast<double>(s1[r]);
            m += static_cast<double>(s2[r]);
            m += static_cast<double>(s3[r]);
            m *= inv_n;
            sq = fma(m, m, sq);
            const double b = m * static_cast<double>(wk[r]);
            acc0 = __builtin_amdgcn_mfma_f64_16x16x4f64(wr[r], b, acc0, 0, 0, 0);
            acc1 = __builtin_amdgcn_mfma_f64_16x16x4f64(wp[r], b, acc1, 0, 0, 0);
        }
    }
    {
        double x[4];
        gather_rows(sq, x);
        sq = ((x[0] + x[1]) + x[2]) + x[3];
    }
    if constexpr (BC) __syncthreads();  // every wave is done with the projection block the tiles overwrite
#pragma unroll
    for (int v = 0; v < 4; ++v) {
        part[wave][0][v][l] = acc0[v];
        part[wave][1][v][l] = acc1[v];
    }
    part_sq[wave][l] = sq;
    __syncthreads();

    // Coefficients, one matrix entry per lane: wave w maps tokens
    // 4w .. 4w+3, lane l -> token tt = 4w + l / 16, entry e = l % 16 (res row
    // e / 4, column e % 4); lanes e < 8 also map pre[e] (e < 4) or
    // post[e - 4]. Partial tiles are summed in wave order, as the same value
    // in every wave.
    const int tt = 4 * wave + l / 16;
    const int e = l % 16;
    const int64_t token_e = static_cast<int64_t>(blockIdx.x) * 16 + tt;
    const bool valid_e = token_e < a.tokens;
    const double sq_tt = ((part_sq[0][tt] + part_sq[1][tt]) + part_sq[2][tt]) + part_sq[3][tt];
    const double scale = 1.0 / sqrt(sq_tt / static_cast<double>(D) + a.eps);
    const int src_res = tt + 16 * (e / 4);            // accumulator lane of res entry e (tile 0, v = e % 4)
    const int src_pp = tt + 16 * (e < 4 ? 0 : 1);     // pre in lane q = 0, post in q = 1 (tile 1, v = e % 4)
    const int v = e % 4;
    const double logit_res =
        ((part[0][0][v][src_res] + part[1][0][v][src_res]) + part[2][0][v][src_res]) + part[3][0][v][src_res];
    const double logit_pp =
        ((part[0][1][v][src_pp] + part[1][1][v][src_pp]) + part[2][1][v][src_pp]) + part[3][1][v][src_pp];
    const double th_res = tanh_d(logit_res * scale);
    const double th_pp = tanh_d(logit_pp * scale);
    double m = exp_d(fma(static_cast<double>(res_alpha), th_res, static_cast<double>(res_bias_e)));
    const bool is_pre = e < 4;
    const float c = static_cast<float>((is_pre ? 1.0 : 2.0) *
                                       sigmoid_fast(fma(static_cast<double>(pp_alpha), th_pp,
                                                        static_cast<double>(pp_bias))));
    // The res chain (tanh, exp) runs here beside the pre/post chain; left to
    // itself the compiler sinks it past the barrier, after the agg pass.
    asm volatile("" : "+v"(m));
    if (e < 8) {
        if (is_pre) pre_lds[tt][v] = c;
        if (valid_e) store_f<NTS>((is_pre ? a.pre : a.post) + token_e * n + v, c);
    }
    __syncthreads();

    // agg = sum_i pre_i * s_i over this wave's k set for its 16 tokens
    // (lane (t, q) layout of the loads): exact products, one rounding.
    double p[n];
#pragma unroll
    for (int i = 0; i < n; ++i) p[i] = static_cast<double>(pre_lds[t][i]);
    float4 aggv[GW];
    double asq = 0.0;
#pragma unroll
    for (int j = 0; j < GW; ++j) {
        float o[4];
        const float s0[4] = {sv[j][0].x, sv[j][0].y, sv[j][0].z, sv[j][0].w};
        const float s1[4] = {sv[j][1].x, sv[j][1].y, sv[j][1].z, sv[j][1].w};
        const float s2[4] = {sv[j][2].x, sv[j][2].y, sv[j][2].z, sv[j][2].w};
        const float s3[4] = {sv[j][3].x, sv[j][3].y, sv[j][3].z, sv[j][3].w};
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            double acc = p[0] * static_cast<double>(s0[r]);
            acc = fma(p[1], static_cast<double>(s1[r]), acc);
            acc = fma(p[2], static_cast<double>(s2[r]), acc);
            acc = fma(p[3], static_cast<double>(s3[r]), acc);
            o[r] = static_cast<float>(acc);
            asq = fma(static_cast<double>(o[r]), static_cast<double>(o[r]), asq);
        }
        aggv[j] = make_float4(o[0], o[1], o[2], o[3]);
    }
    float* agg_row = a.agg + (valid ? token : 0) * D;
    if (a.agg_norm_w != nullptr) {
        double x[4];
        gather_rows(asq, x);
        asq = ((x[0] + x[1]) + x[2]) + x[3];
        agg_sq[wave][l] = asq;
        __syncthreads();
        const double total = ((agg_sq[0][l] + agg_sq[1][l]) + agg_sq[2][l]) + agg_sq[3][l];
        const double ascale = 1.0 / sqrt(total / static_cast<double>(D) + a.agg_norm_eps);
#pragma unroll
        for (int j = 0; j < GW; ++j) {
            const float4 w4 = anw[j];
            float4& o = aggv[j];
            o.x = static_cast<float>((static_cast<double>(o.x) * ascale) * static_cast<double>(w4.x));
            o.y = static_cast<float>((static_cast<double>(o.y) * ascale) * static_cast<double>(w4.y));
            o.z = static_cast<float>((static_cast<double>(o.z) * ascale) * static_cast<double>(w4.z));
            o.w = static_cast<float>((static_cast<double>(o.w) * ascale) * static_cast<double>(w4.w));
        }
    }
    if (valid) {
#pragma unroll
        for (int j = 0; j < GW; ++j) {
            store_f4<NTS>(agg_row + 16 * (wave * GW + j) + 4 * q, aggv[j]);
        }
    }

    // Sinkhorn, one entry per lane (token tt, entry e): row sums over the quad,
    // column sums over the 16-lane group, reciprocals then products as in the
    // reference (1 / s, then m * (1 / s)).
    // Only a first-round row sum can be infinite: after a row normalisation
    // every entry is at most 1 (+1 ulp), so later sums stay below 5. When no
    // entry of the wave reaches 2^1020, four of them cannot overflow and the
    // loop runs without the reciprocal's infinity test (same results).
    const int rounds = a.iters > 1 ? a.iters : 1;
    if (__all(m < 0x1p1020)) {
        for (int it = 0; it < rounds; ++it) {
            m *= recip_finite(quad_sum(m));
            m *= recip_finite(column_sum(m));
        }
    } else {
        for (int it = 0; it < rounds; ++it) {
            m *= recip_pos(quad_sum(m));
            m *= recip_pos(column_sum(m));
        }
    }
    if (valid_e) store_f<NTS>(a.res + token_e * 16 + e, static_cast<float>(m));
}

// ---------------------------------------------------------------------------
// prepare, generic path: one wave per token, reference association
// ---------------------------------------------------------------------------

struct GenericArgs {
    PrepareArgs p;
    int n;
    int64_t d;
};

__global__ __launch_bounds__(kWave) void mhc_prepare_generic_kernel(GenericArgs g) {
    extern __shared__ double smem[];
    const PrepareArgs& a = g.p;
    const int n = g.n;
    const int64_t d = g.d;
    const int rows = 2 * n + n * n;
    double* ref = smem;                 // [d]
    double* logit = ref + d;            // [rows]
    double* mat = logit + rows;         // [n*n]
    double* sums = mat + n * n;         // [n]
    float* pref = reinterpret_cast<float*>(sums + n);  // [n]
    float* aggf = pref + n;                             // [d]
    const int lane = threadIdx.x;
    const int64_t token = blockIdx.x;
    const float* s = a.streams + token * a.ts;
    const double inv_n = 1.0 / static_cast<double>(n);

    for (int64_t k = lane; k < d; k += kWave) {
        double m = static_cast<double>(s[k]);
        for (int i = 1; i < n; ++i) m += static_cast<double>(s[i * a.sd + k]);
        ref[k] = m * inv_n;
    }
    __syncthreads();
    __shared__ double scale_s;
    if (lane == 0) {
        // Four double lanes over the 4-aligned part, hsum, scalar tail.
        double sq[4] = {0.0, 0.0, 0.0, 0.0};
        int64_t k = 0;
        for (; k + 4 <= d; k += 4) {
            for (int v = 0; v < 4; ++v) sq[v] = fma(ref[k + v], ref[k + v], sq[v]);
        }
        double sumsq = (sq[0] + sq[1]) + (sq[2] + sq[3]);
        for (; k < d; ++k) sumsq = fma(ref[k], ref[k], sumsq);
        scale_s = 1.0 / sqrt(sumsq / static_cast<double>(d) + a.eps);
    }
    __syncthreads();
    const double scale = scale_s;
    for (int64_t k = lane; k < d; k += kWave) ref[k] = (ref[k] * scale) * static_cast<double>(a.norm_w[k]);
    __syncthreads();
    for (int r = lane; r < rows; r += kWave) {
        const double* w = a.proj_w + static_cast<int64_t>(r) * d;
        double acc[4] = {0.0, 0.0, 0.0, 0.0};
        int64_t k = 0;
        for (; k + 4 <= d; k += 4) {
            for (int v = 0; v < 4; ++v) acc[v] = fma(w[k + v], ref[k + v], acc[v]);
        }
        double out = (acc[0] + acc[1]) + (acc[2] + acc[3]);
        for (; k < d; ++k) out = fma(w[k], ref[k], out);
        logit[r] = tanh(out);
    }
    __syncthreads();
    const double pre_alpha = static_cast<double>(*a.pre_alpha);
    const double post_alpha = static_cast<double>(*a.post_alpha);
    const double res_alpha = static_cast<double>(*a.res_alpha);
    for (int i = lane; i < n; i += kWave) {
        pref[i] = static_cast<float>(sigmoid_d(fma(pre_alpha, logit[i], static_cast<double>(a.pre_bias[i]))));
        a.pre[token * n + i] = pref[i];
        a.post[token * n + i] =
            static_cast<float>(2.0 * sigmoid_d(fma(post_alpha, logit[n + i], static_cast<double>(a.post_bias[i]))));
    }
    for (int e = lane; e < n * n; e += kWave) {
        mat[e] = fma(res_alpha, logit[2 * n + e], static_cast<double>(a.res_bias[e]));
    }
    __syncthreads();
    for (int64_t k = lane; k < d; k += kWave) {
        double acc = static_cast<double>(pref[0]) * static_cast<double>(s[k]);
        for (int i = 1; i < n; ++i) {
            acc = fma(static_cast<double>(pref[i]), static_cast<double>(s[i * a.sd + k]), acc);
        }
        aggf[k] = static_cast<float>(acc);
    }
    __syncthreads();
    if (lane == 0) {
        if (a.agg_norm_w != nullptr) {
            double acc0[4] = {0, 0, 0, 0}, acc1[4] = {0, 0, 0, 0};
            int64_t k = 0;
            for (; k + 8 <= d; k += 8) {
                for (int v = 0; v < 4; ++v) {
                    const double x0 = aggf[k + v], x1 = aggf[k + 4 + v];
                    acc0[v] = fma(x0, x0, acc0[v]);
                    acc1[v] = fma(x1, x1, acc1[v]);
                }
            }
            double tv[4];
            for (int v = 0; v < 4; ++v) tv[v] = acc0[v] + acc1[v];
            double sumsq = (tv[0] + tv[1]) + (tv[2] + tv[3]);
            for (; k < d; ++k) sumsq = fma(static_cast<double>(aggf[k]), static_cast<double>(aggf[k]), sumsq);
            scale_s = 1.0 / sqrt(sumsq / static_cast<double>(d) + a.agg_norm_eps);
        }
        // Sinkhorn in the reference's order.
        for (int e = 0; e < n * n; ++e) mat[e] = exp(mat[e]);
        const int rounds = a.iters > 1 ? a.iters : 1;
        for (int it = 0; it < rounds; ++it) {
            for (int i = 0; i < n; ++i) {
                double sum = mat[i * n];
                for (int j = 1; j < n; ++j) sum += mat[i * n + j];
                const double inv = 1.0 / sum;
                for (int j = 0; j < n; ++j) mat[i * n + j] *= inv;
            }
            for (int j = 0; j < n; ++j) {
                double sum = mat[j];
                for (int i = 1; i < n; ++i) sum += mat[i * n + j];
                sums[j] = 1.0 / sum;
            }
            for (int i = 0; i < n; ++i) {
                for (int j = 0; j < n; ++j) mat[i * n + j] *= sums[j];
            }
        }
    }
    __syncthreads();
    for (int e = lane; e < n * n; e += kWave) a.res[token * n * n + e] = static_cast<float>(mat[e]);
    const double ascale = scale_s;
    for (int64_t k = lane; k < d; k += kWave) {
        float v = aggf[k];
        if (a.agg_norm_w != nullptr) {
            v = static_cast<float>((static_cast<double>(v) * ascale) * static_cast<double>(a.agg_norm_w[k]));
        }
        a.agg[token * d + k] = v;
    }
}

// ---------------------------------------------------------------------------
// combine
// ---------------------------------------------------------------------------

// I: index type of the flat (token, 4-column chunk) index; 32-bit when it fits,
// which keeps the per-thread division by the chunk count cheap.
// CPT 16-byte chunks per thread, d / CPT apart (CPT = 2 for n = 4: the
// token's coefficients fetched once for twice the work and twice the loads in
// flight; 8.3 -> 7.85 us at 8192 tokens, d = 128).
template <int N, typename I, int CPT = 1>
// streams and new_streams may be one buffer (in place): a thread writes exactly
// the stream elements it has read, and every new value depends on all of them.
__global__ __launch_bounds__(kBlock) void mhc_combine_vec_kernel(const float* streams, int64_t tokens,
                                                                 int64_t d, int64_t sd, int64_t ts,
                                                                 const float* __restrict__ res,
                                                                 const float* __restrict__ post,
                                                                 const float* __restrict__ out,
                                                                 float* new_streams,
                                                                 float* __restrict__ collapsed) {
    const I chunks = static_cast<I>(d / 4 / CPT);
    const I idx = static_cast<I>(blockIdx.x) * kBlock + threadIdx.x;
    if (static_cast<int64_t>(idx) >= tokens * static_cast<int64_t>(chunks)) return;
    const I token_i = idx / chunks;
    const int64_t token = token_i;
    const int64_t k0 = static_cast<int64_t>(idx - token_i * chunks) * 4;
    float4 oc[CPT], sc[CPT][N];
#pragma unroll
    for (int c = 0; c < CPT; ++c) {
        const int64_t k = k0 + c * (d / CPT);
        oc[c] = *reinterpret_cast<const float4*>(out + token * d + k);
#pragma unroll
        for (int j = 0; j < N; ++j) {
            const nt_f4 x = __builtin_nontemporal_load(reinterpret_cast<const nt_f4*>(streams + token * ts + j * sd + k));
            sc[c][j] = make_float4(x[0], x[1], x[2], x[3]);
        }
    }
    // The token's coefficients: shared by every thread of the token, fetched
    // as whole 16-byte rows when n = 4 (one request per row, not per value).
    float rv[N * N], pv[N];
    if constexpr (N == 4) {
        const float4* r4 = reinterpret_cast<const float4*>(res + token * 16);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const float4 x = r4[i];
            rv[4 * i] = x.x;
            rv[4 * i + 1] = x.y;
            rv[4 * i + 2] = x.z;
            rv[4 * i + 3] = x.w;
        }
        const float4 y = *reinterpret_cast<const float4*>(post + token * 4);
        pv[0] = y.x;
        pv[1] = y.y;
        pv[2] = y.z;
        pv[3] = y.w;
    } else {
#pragma unroll
        for (int i = 0; i < N * N; ++i) rv[i] = res[token * N * N + i];
#pragma unroll
        for (int i = 0; i < N; ++i) pv[i] = post[token * N + i];
    }
#pragma unroll
    for (int c = 0; c < CPT; ++c) {
        const int64_t k = k0 + c * (d / CPT);
        const float4 o = oc[c];
        const float4* s = sc[c];
        double mean[4] = {0.0, 0.0, 0.0, 0.0};
#pragma unroll
        for (int i = 0; i < N; ++i) {
            const double pi = static_cast<double>(pv[i]);
            double acc[4] = {pi * o.x, pi * o.y, pi * o.z, pi * o.w};
#pragma unroll
            for (int j = 0; j < N; ++j) {
                const double rij = static_cast<double>(rv[i * N + j]);
                acc[0] = fma(rij, static_cast<double>(s[j].x), acc[0]);
                acc[1] = fma(rij, static_cast<double>(s[j].y), acc[1]);
                acc[2] = fma(rij, static_cast<double>(s[j].z), acc[2]);
                acc[3] = fma(rij, static_cast<double>(s[j].w), acc[3]);
            }
            const float4 nv = make_float4(static_cast<float>(acc[0]), static_cast<float>(acc[1]),
                                          static_cast<float>(acc[2]), static_cast<float>(acc[3]));
            if (new_streams != nullptr) {
                const nt_f4 x = {nv.x, nv.y, nv.z, nv.w};
                __builtin_nontemporal_store(x, reinterpret_cast<nt_f4*>(new_streams + (token * N + i) * d + k));
            }
            mean[0] += static_cast<double>(nv.x);
            mean[1] += static_cast<double>(nv.y);
            mean[2] += static_cast<double>(nv.z);
            mean[3] += static_cast<double>(nv.w);
        }
        if (collapsed != nullptr) {
            const double inv_n = 1.0 / static_cast<double>(N);
            *reinterpret_cast<float4*>(collapsed + token * d + k) =
                make_float4(static_cast<float>(mean[0] * inv_n), static_cast<float>(mean[1] * inv_n),
                            static_cast<float>(mean[2] * inv_n), static_cast<float>(mean[3] * inv_n));
        }
    }
}

// Any n, d, stride and alignment: one thread per (token, k). The token's n
// old stream values at k are read before any new one is stored (n <= 8 in
// registers), so streams and new_streams may be one buffer.
template <typename I>
__global__ __launch_bounds__(kBlock) void mhc_combine_scalar_kernel(const float* streams,
                                                                    int64_t tokens, int n, int64_t d, int64_t sd,
                                                                    int64_t ts, const float* __restrict__ res,
                                                                    const float* __restrict__ post,
                                                                    const float* __restrict__ out,
                                                                    float* new_streams,
                                                                    float* __restrict__ collapsed) {
    const I idx = static_cast<I>(blockIdx.x) * kBlock + threadIdx.x;
    if (static_cast<int64_t>(idx) >= tokens * d) return;
    const I token_i = idx / static_cast<I>(d);
    const int64_t token = token_i;
    const int64_t k = idx - token_i * static_cast<I>(d);
    const double o = static_cast<double>(out[token * d + k]);
    const float* s = streams + token * ts + k;
    constexpr int kMax = 8;
    double old[kMax];
    const bool held = n <= kMax;
#pragma unroll
    for (int j = 0; j < kMax; ++j) old[j] = held && j < n ? static_cast<double>(s[j * sd]) : 0.0;
    double mean = 0.0;
    for (int i = 0; i < n; ++i) {
        double acc = static_cast<double>(post[token * n + i]) * o;
        if (held) {
#pragma unroll
            for (int j = 0; j < kMax; ++j) {
                if (j < n) acc = fma(static_cast<double>(res[(token * n + i) * n + j]), old[j], acc);
            }
        } else {
            for (int j = 0; j < n; ++j) {
                acc = fma(static_cast<double>(res[(token * n + i) * n + j]), static_cast<double>(s[j * sd]), acc);
            }
        }
        const float nv = static_cast<float>(acc);
        if (new_streams != nullptr) new_streams[(token * n + i) * d + k] = nv;
        mean += static_cast<double>(nv);
    }
    if (collapsed != nullptr) collapsed[token * d + k] = static_cast<float>(mean * (1.0 / static_cast<double>(n)));
}

mlk_status launch_combine(const float* streams, int64_t tokens, int64_t n, int64_t d, int64_t sd, int64_t ts,
                          const float* res, const float* post, const float* out, float* new_streams,
                          float* collapsed, hipStream_t stream) {
    if (tokens == 0) return MLK_OK;
    auto al16 = [](const void* p) { return p == nullptr || reinterpret_cast<uintptr_t>(p) % 16 == 0; };
    const bool vec = d % 4 == 0 && sd % 4 == 0 && ts % 4 == 0 && al16(streams) && al16(out) && al16(new_streams) &&
                     al16(collapsed) && n >= 1 && n <= 8 && (n != 4 || (al16(res) && al16(post)));
    if (vec) {
        const int64_t blocks = ceil_div(tokens * (d / 4), kBlock);
        // Two chunks per thread when the new streams are written (the collapse
        // alone measured slower with them: 273 -> 286 us at 262144 tokens, d 256).
        if (n == 4 && new_streams != nullptr && d % 8 == 0 && tokens * (d / 8) < (int64_t{1} << 31)) {
            hipLaunchKernelGGL((mhc_combine_vec_kernel<4, uint32_t, 2>), dim3(ceil_div(tokens * (d / 8), kBlock)), dim3(kBlock), 0,
                               stream, streams, tokens, d, sd, ts, res, post, out, new_streams, collapsed);
            return launch_status("mhc_combine");
        }
        const bool narrow = tokens * (d / 4) < (int64_t{1} << 31);
#define MLK_COMBINE(NN)                                                                                        \
    case NN:                                                                                                   \
        if (narrow) {                                                                                          \
            hipLaunchKernelGGL((mhc_combine_vec_kernel<NN, uint32_t>), dim3(blocks), dim3(kBlock), 0, stream,  \
                               streams, tokens, d, sd, ts, res, post, out, new_streams, collapsed);            \
        } else {                                                                                               \
            hipLaunchKernelGGL((mhc_combine_vec_kernel<NN, int64_t>), dim3(blocks), dim3(kBlock), 0, stream,   \
                               streams, tokens, d, sd, ts, res, post, out, new_streams, collapsed);            \
        }                                                                                                      \
        break;
        switch (n) {
            MLK_COMBINE(1)
            MLK_COMBINE(2)
            MLK_COMBINE(3)
            MLK_COMBINE(4)
            MLK_COMBINE(5)
            MLK_COMBINE(6)
            MLK_COMBINE(7)
            MLK_COMBINE(8)
            default: break;
        }
#undef MLK_COMBINE
        return launch_status("mhc_combine");
    }
    const int64_t blocks = ceil_div(tokens * d, kBlock);
    if (tokens * d < (int64_t{1} << 31)) {
        hipLaunchKernelGGL(mhc_combine_scalar_kernel<uint32_t>, dim3(blocks), dim3(kBlock), 0, stream, streams,
                           tokens, static_cast<int>(n), d, sd, ts, res, post, out, new_streams, collapsed);
    } else {
        hipLaunchKernelGGL(mhc_combine_scalar_kernel<int64_t>, dim3(blocks), dim3(kBlock), 0, stream, streams,
                           tokens, static_cast<int>(n), d, sd, ts, res, post, out, new_streams, collapsed);
    }
    return launch_status("mhc_combine");
}

// The streams may be overwritten in place (new_streams == streams) when they
// are contiguous [tokens, n, d] and n <= 8 (the combine kernels then hold a
// token's old values at each k before storing the new ones; the fused combine
// + prepare kernel reads everything a token needs before its first barrier
// and stores after it).
bool in_place_ok(int64_t n, int64_t d, int64_t sd, int64_t ts) { return n <= 8 && sd == d && ts == n * d; }

bool prepare_fast(const PrepareArgs& a, int64_t n, int64_t d) {
    auto al16 = [](const void* p) { return p == nullptr || reinterpret_cast<uintptr_t>(p) % 16 == 0; };
    return n == 4 && (d == 64 || d == 128 || d == 256 || d == 512) && a.sd % 4 == 0 && a.ts % 4 == 0 &&
           al16(a.streams) && al16(a.norm_w) && al16(a.agg_norm_w) && al16(a.agg) && al16(a.pre) && al16(a.post) &&
           al16(a.res) && al16(a.proj_w);
}

// The fused combine + prepare kernel: n = 4, d <= 256 (d = 512 has no
// registers to spare), every operand 16-byte aligned.
bool prepare_fusable(const PrepareArgs& a, int64_t n, int64_t d) {
    auto al16 = [](const void* p) { return reinterpret_cast<uintptr_t>(p) % 16 == 0; };
    return prepare_fast(a, n, d) && d <= 256 && al16(a.c_res) && al16(a.c_post) && al16(a.c_out) && al16(a.c_new);
}

mlk_status launch_prepare(const PrepareArgs& a, int64_t n, int64_t d, hipStream_t stream, bool fused = false) {
    if (a.tokens == 0) return MLK_OK;
    if (fused || prepare_fast(a, n, d)) {
        const int64_t blocks = ceil_div(a.tokens, 16);
        // Non-temporal output stores, except in the fused combine + prepare above 65,536 tokens (measured:
        // 262,144 tokens at d 256 take 0.61 instead of 0.68 ms with plain stores there, while the plain
        // form of the prepare alone is slower, 0.35 against 0.33 ms, and 8,192 tokens gain from
        // non-temporal stores).
        const bool nts = a.tokens <= 65536;
#define MLK_PREP_NTS(DV, F)                                                                                       \
    if (nts) {                                                                                                    \
        hipLaunchKernelGGL((mhc_prepare_n4_kernel<DV, F, true>), dim3(blocks), dim3(kBlock), 0, stream, a);       \
    } else {                                                                                                      \
        hipLaunchKernelGGL((mhc_prepare_n4_kernel<DV, F, false>), dim3(blocks), dim3(kBlock), 0, stream, a);      \
    }
#define MLK_PREP(DV)                                                                                              \
    case DV:                                                                                                      \
        if (fused) {                                                                                              \
            MLK_PREP_NTS((DV <= 256 ? DV : 256), true)                                                            \
        } else {                                                                                                  \
            if (a.sd == 0 && (DV == 128 || DV == 256)) {                                                          \
                hipLaunchKernelGGL((mhc_prepare_n4_kernel<DV, false, true, (DV == 128 || DV == 256)>),            \
                                   dim3(blocks),                                                                  \
                                   dim3(kBlock), 0, stream, a);                                                   \
            } else {                                                                                              \
                hipLaunchKernelGGL((mhc_prepare_n4_kernel<DV, false, true>), dim3(blocks), dim3(kBlock), 0,       \
                                   stream, a);                                                                    \
            }                                                                                                     \
        }                                                                                                         \
        break;
        switch (d) {
            MLK_PREP(64)
            MLK_PREP(128)
            MLK_PREP(256)
            MLK_PREP(512)
            default: break;
        }
#undef MLK_PREP
#undef MLK_PREP_NTS
        return launch_status("mhc_prepare");
    }
    GenericArgs g{a, static_cast<int>(n), d};
    const size_t shmem = sizeof(double) * static_cast<size_t>(d + 2 * n + 2 * n * n + n) + sizeof(float) * (d + n);
    if (shmem > 64 * 1024) {
        set_error("mhc_prepare: d too large for the generic path");
        return MLK_ERR_UNSUPPORTED;
    }
    hipLaunchKernelGGL(mhc_prepare_generic_kernel, dim3(a.tokens), dim3(kWave), shmem, stream, g);
    return launch_status("mhc_prepare");
}

mlk_status check_prepare(int64_t tokens, int64_t n, int64_t d, const double* proj_w, int64_t iters) {
    MLK_CHECK(n > 0 && d > 0, "streams must be non-empty");
    MLK_CHECK(iters >= 0, "sinkhorn_iters must be non-negative");
    MLK_CHECK(tokens >= 0, "streams must be [B,L,n,d] or a broadcast [B,L,d]");
    MLK_CHECK(tokens == 0 || proj_w != nullptr, "proj_w must be [2n + n*n, d]");
    return MLK_OK;
}

}  // namespace
}  // namespace mlk

using namespace mlk;

extern "C" {

mlk_status mlk_mhc_prepare(const float* streams, int64_t tokens, int64_t n, int64_t d, int64_t stream_stride,
                           int64_t token_stride, const float* norm_w, double eps, const double* proj_w,
                           const float* pre_bias, const float* post_bias, const float* res_bias,
                           const float* pre_alpha, const float* post_alpha, const float* res_alpha,
                           int64_t sinkhorn_iters, const float* agg_norm_w, double agg_norm_eps, float* agg,
                           float* pre, float* post, float* res, mlk_stream_t stream) {
    const mlk_status st = check_prepare(tokens, n, d, proj_w, sinkhorn_iters);
    if (st != MLK_OK) return st;
    PrepareArgs a{};
    a.streams = streams;
    a.tokens = tokens;
    a.sd = stream_stride;
    a.ts = token_stride;
    a.norm_w = norm_w;
    a.eps = static_cast<double>(static_cast<float>(eps));
    a.proj_w = proj_w;
    a.pre_bias = pre_bias;
    a.post_bias = post_bias;
    a.res_bias = res_bias;
    a.pre_alpha = pre_alpha;
    a.post_alpha = post_alpha;
    a.res_alpha = res_alpha;
    a.iters = static_cast<int>(sinkhorn_iters < (1 << 20) ? sinkhorn_iters : (1 << 20));
    a.agg_norm_w = agg_norm_w;
    a.agg_norm_eps = static_cast<double>(static_cast<float>(agg_norm_eps));
    a.agg = agg;
    a.pre = pre;
    a.post = post;
    a.res = res;
    return launch_prepare(a, n, d, stream);
}

mlk_status mlk_mhc_combine(const float* streams, int64_t tokens, int64_t n, int64_t d, int64_t stream_stride,
                           int64_t token_stride, const float* res, const float* post, const float* out,
                           float* new_streams, float* collapsed, mlk_stream_t stream) {
    MLK_CHECK(n > 0 && d > 0, "streams must be non-empty");
    MLK_CHECK(new_streams != nullptr || collapsed != nullptr || tokens == 0, "mhc_combine needs an output");
    MLK_CHECK(new_streams != streams || in_place_ok(n, d, stream_stride, token_stride),
              "in-place mhc_combine needs contiguous [tokens, n, d] streams and n <= 8");
    if (tokens == 0) return MLK_OK;
    return launch_combine(streams, tokens, n, d, stream_stride, token_stride, res, post, out, new_streams, collapsed,
                          stream);
}

mlk_status mlk_mhc_combine_prepare(const float* streams, int64_t tokens, int64_t n, int64_t d,
                                   int64_t stream_stride, int64_t token_stride, const float* res, const float* post,
                                   const float* out, const float* norm_w, double eps, const double* proj_w,
                                   const float* pre_bias, const float* post_bias, const float* res_bias,
                                   const float* pre_alpha, const float* post_alpha, const float* res_alpha,
                                   int64_t sinkhorn_iters, const float* agg_norm_w, double agg_norm_eps,
                                   float* new_streams, float* agg_out, float* pre_out, float* post_out,
                                   float* res_out, mlk_stream_t stream) {
    MLK_CHECK(new_streams != nullptr || tokens == 0, "new_streams must be given");
    MLK_CHECK(new_streams != streams || in_place_ok(n, d, stream_stride, token_stride),
              "in-place mhc_combine_prepare needs contiguous [tokens, n, d] streams and n <= 8");
    mlk_status st = check_prepare(tokens, n, d, proj_w, sinkhorn_iters);
    if (st != MLK_OK) return st;
    if (tokens == 0) return MLK_OK;
    // n = 4 and d <= 256: one kernel writes the new streams and prepares the
    // next residual from them in registers (the new streams are not read back).
    PrepareArgs a{};
    a.streams = streams;
    a.tokens = tokens;
    a.sd = stream_stride;
    a.ts = token_stride;
    a.norm_w = norm_w;
    a.eps = static_cast<double>(static_cast<float>(eps));
    a.proj_w = proj_w;
    a.pre_bias = pre_bias;
    a.post_bias = post_bias;
    a.res_bias = res_bias;
    a.pre_alpha = pre_alpha;
    a.post_alpha = post_alpha;
    a.res_alpha = res_alpha;
    a.iters = static_cast<int>(sinkhorn_iters < (1 << 20) ? sinkhorn_iters : (1 << 20));
    a.agg_norm_w = agg_norm_w;
    a.agg_norm_eps = static_cast<double>(static_cast<float>(agg_norm_eps));
    a.agg = agg_out;
    a.pre = pre_out;
    a.post = post_out;
    a.res = res_out;
    a.c_res = res;
    a.c_post = post;
    a.c_out = out;
    a.c_new = new_streams;
    if (prepare_fusable(a, n, d)) {
        MLK_CHECK(res && post && out, "null tensor pointer");
        return launch_prepare(a, n, d, stream, true);
    }
    st = launch_combine(streams, tokens, n, d, stream_stride, token_stride, res, post, out, new_streams, nullptr,
                        stream);
    if (st != MLK_OK) return st;
    return mlk_mhc_prepare(new_streams, tokens, n, d, d, n * d, norm_w, eps, proj_w, pre_bias, post_bias, res_bias,
                           pre_alpha, post_alpha, res_alpha, sinkhorn_iters, agg_norm_w, agg_norm_eps, agg_out,
                           pre_out, post_out, res_out, stream);
}

}  // extern "C"
