// Mamba-3 SISO mixer on gfx950: the in_proj post-processing (phases A, B, C)
// and the trapezoidal recurrence, plus the one-token step with carried state.
//
// Reference semantics: rdt4quant_cpu/montlok_kernel.h (prep :463-597,
// recurrence :251-457), rdt4quant_cpu/montlok_types.h (softplus, sigmoid,
// heavy_tail, step_coefficients :57-93), op glue rdt4quant_cpu/montlok.cpp
// (:245-492).
//
// in_proj row layout [z | x | B | C | dt | A | trap | angles], widths
// [d_inner, d_inner, G*N, G*N, H, H, H, R].
//
// Kernels
//   prep_kernel     one thread per (token, head): BCNorm of the head's B and C
//                   group (fp32, sequential sum), biases -> unrotated k, q;
//                   dt/A/trap -> (alpha, beta, gamma); tanh(angle)*pi*dt.
//   rotate_kernel   one thread per (window, head, angle r): the running angle
//                   sum over time in double, rounded to fp32 per step, wrapped
//                   to [0, 2pi) with a separately rounded 2pi*floor product,
//                   sin/cos in double, rotation of pair (2r, 2r+1) of q and k.
//   rec_kernel<NM>  the time-sequential recurrence: one wave per (window,
//                   head, 64 headdim columns), lane d owns state column S[:, d]
//                   (N <= NM floats in VGPRs); q_t, k_t, k_{t-1}, the
//                   coefficients, v and the gate of 8-step chunks are staged in
//                   LDS, double-buffered. Per step and state row n:
//                     s = fma(k_t[n], gamma*v_t[d], fma(s, alpha, k_{t-1}[n] * beta*v_{t-1}[d]))
//                     acc_{n%2} = fma(s, q_t[n], acc)
//                   (even/odd accumulators when headdim % 8 == 0, one
//                   otherwise, as the reference's vector and scalar paths),
//                   y = fma(D, v_t[d], acc0 + acc1), out = y * silu(z) in double
//                   rounded once (or y * gate). Bit for bit the reference's
//                   association; fp32-VALU bound, ~7 flop per state element
//                   per token.
//   rec_chunk_kernel the chunked scan on the fp32 matrix cores (32-token
//                   chunks, state carried in registers), used by the
//                   recurrent op when there are few (window, head) pairs; see
//                   the comment above it.
//   scan_fused_kernel the forward in one kernel: the prep and rotate steps
//                   above and rec_chunk_kernel's scan per (window, head)
//                   straight from the in_proj rows, q and k kept in LDS; the
//                   forward's default for d_state 16/32/64, headdim 16/32/64.
#include <cstdlib>
#include <cstring>
#include <type_traits>

#include <mutex>

#include "mlk_common.h"
#include "tile_f32.h"

namespace mlk {
namespace {

constexpr float kPiF = 3.14159265358979323846f;
constexpr float kTwoPiF = 6.28318530717958647692f;

// fp32 exp / log1p / tanh evaluated in double and rounded once: the
// correctly rounded value except in rare double-rounding cases, which is what
// the host libm the reference links (glibc) returns for these functions.
__device__ __forceinline__ float expf_cr(float x) { return static_cast<float>(exp_d(static_cast<double>(x))); }
__device__ __forceinline__ float log1pf_cr(float x) { return static_cast<float>(log1p(static_cast<double>(x))); }
__device__ __forceinline__ float tanhf_cr(float x) { return static_cast<float>(tanh_d(static_cast<double>(x))); }

// base[elem_off] with the byte offset formed in 32 bits: the load can then take a scalar base and a 32-bit
// vector offset, with no 64-bit address add per load (elem_off * 4 < 2^32 at every call).
__device__ __forceinline__ float load_off32(const float* base, unsigned elem_off) {
    return *reinterpret_cast<const float*>(reinterpret_cast<const char*>(base) + (elem_off << 2));
}
__device__ __forceinline__ void store_off32(float* base, unsigned elem_off, float v) {
    *reinterpret_cast<float*>(reinterpret_cast<char*>(base) + (elem_off << 2)) = v;
}

// torch softplus (beta 1, threshold 20) as montlok_types.h:58-60 evaluates it.
__device__ __forceinline__ float softplus_f(float x) { return x > 20.0f ? x : log1pf_cr(expf_cr(x)); }
__device__ __forceinline__ float sigmoid_f(float x) { return 1.0f / (1.0f + expf_cr(-x)); }
__device__ __forceinline__ float heavy_tail_f(float x) {
    const float negative = fminf(x, 0.0f);
    const float positive = fmaxf(x, 0.0f);
    return positive + 1.0f / (1.0f - negative);
}

// (alpha, beta, gamma) = (exp(adt), (1 - sig(trap)) * dt * alpha, sig(trap) * dt).
__device__ __forceinline__ void step_coefficients(float adt, float dt, float trap_logit, float* alpha, float* beta,
                                                  float* gamma) {
    const float a = expf_cr(adt);
    const float trap = sigmoid_f(trap_logit);
    *alpha = a;
    *beta = ((1.0f - trap) * dt) * a;
    *gamma = trap * dt;
}

// BCNorm scale of one group (montlok_kernel.h:464-474): sequential fp32 sum of
// squares, each square of the first 4*floor(n/4) elements rounded before the
// add and the remainder fused, as the compiled reference evaluates it.
__device__ __forceinline__ float bc_norm_scale(const float* x, int64_t n, float eps) {
    float ss = 0.0f;
    const int64_t body = n - n % 4;
    for (int64_t i = 0; i < body; ++i) ss = ss + x[i] * x[i];
    for (int64_t i = body; i < n; ++i) ss = fmaf(x[i], x[i], ss);
    return 1.0f / sqrtf(ss / static_cast<float>(n) + eps);
}

// The same sum over x in LDS, read four at a time so the loads batch; the
// additions stay in the same sequential order.
__device__ __forceinline__ float bc_norm_scale_lds(const float* x, int64_t n, float eps) {
    float ss = 0.0f;
    const int64_t body = n - n % 4;
    for (int64_t i = 0; i < body; i += 4) {
        const float a0 = x[i], a1 = x[i + 1], a2 = x[i + 2], a3 = x[i + 3];
        ss = ss + a0 * a0;
        ss = ss + a1 * a1;
        ss = ss + a2 * a2;
        ss = ss + a3 * a3;
    }
    for (int64_t i = body; i < n; ++i) ss = fmaf(x[i], x[i], ss);
    return 1.0f / sqrtf(ss / static_cast<float>(n) + eps);
}

// bc_norm_scale_lds for a compile-time row length N (a multiple of 8), eight
// elements in flight at a time: the same sequential order of additions.
template <int N>
__device__ __forceinline__ float bc_norm_scale_rows(const float* x, float eps) {
    static_assert(N % 8 == 0, "row length");
    float ss = 0.0f;
#pragma unroll 1
    for (int i = 0; i < N; i += 8) {
        const float4 u = *reinterpret_cast<const float4*>(x + i);
        const float4 w = *reinterpret_cast<const float4*>(x + i + 4);
        ss = ss + u.x * u.x;
        ss = ss + u.y * u.y;
        ss = ss + u.z * u.z;
        ss = ss + u.w * u.w;
        ss = ss + w.x * w.x;
        ss = ss + w.y * w.y;
        ss = ss + w.z * w.z;
        ss = ss + w.w * w.w;
    }
    return 1.0f / sqrtf(ss / static_cast<float>(N) + eps);
}

struct PrepArgs {
    const float* proj;
    int64_t sb, st;
    int64_t B, L, N, G, H, D, R;
    const float* b_bias;
    const float* c_bias;
    const float* b_norm_w;
    const float* c_norm_w;
    float b_eps, c_eps;
    const float* dt_bias;
    float a_floor;
    float* q;      // [B, L, H, N]
    float* k;      // [B, L, H, N]
    float* alpha;  // [B, L, H]
    float* beta;
    float* gamma;
    float* term;   // [B, L, H, max(R, 1)]
};

// Phase A for kPrepTokens tokens per block (32 when that still leaves at least
// 1024 blocks, else 8): the [B | C | dt | A | trap | angles] slice of each
// token's row and the B/C norm weights and biases are staged in LDS with
// coalesced loads, then norms (one thread per token and group), coefficients
// (per token and head), q/k (per element) and the angle terms are computed
// from LDS.
template <int kPrepTokens>
__global__ __launch_bounds__(256) void prep_kernel(PrepArgs p) {
    extern __shared__ float seg_s[];
    // Block-local index math in 32 bits (the sizes are checked at launch).
    const int N = static_cast<int>(p.N), G = static_cast<int>(p.G), H = static_cast<int>(p.H);
    const int R = static_cast<int>(p.R);
    const int GN = G * N;
    const int seg = 2 * GN + 3 * H + R;
    const int64_t d_inner = p.H * p.D;
    float* sc_s = seg_s + kPrepTokens * seg;  // [tokens][2G]
    float* dt_s = sc_s + kPrepTokens * 2 * G;  // [tokens][H]
    float* bw_s = dt_s + kPrepTokens * H;      // [N] B norm weight, then [N] C norm weight
    float* bb_s = bw_s + 2 * N;                // [H][N] B bias, then [H][N] C bias
    __shared__ const float* rows_s[kPrepTokens];
    const int64_t BL = p.B * p.L;
    const int64_t tok0 = static_cast<int64_t>(blockIdx.x) * kPrepTokens;
    const int ntok = static_cast<int>(BL - tok0 < kPrepTokens ? BL - tok0 : kPrepTokens);
    const int tid = threadIdx.x;
    if (tid < ntok) {
        const int64_t tok = tok0 + tid;
        rows_s[tid] = p.proj + (tok / p.L) * p.sb + (tok % p.L) * p.st + 2 * d_inner;
    }
    __syncthreads();
    for (int i = tid; i < kPrepTokens * seg; i += 256) {
        const int tt = i / seg, j = i - tt * seg;
        seg_s[i] = tt < ntok ? rows_s[tt][j] : 0.0f;
    }
    for (int i = tid; i < N; i += 256) {
        bw_s[i] = p.b_norm_w[i];
        bw_s[N + i] = p.c_norm_w[i];
    }
    for (int i = tid; i < H * N; i += 256) {
        bb_s[i] = p.b_bias[i];
        bb_s[H * N + i] = p.c_bias[i];
    }
    __syncthreads();
    for (int i = tid; i < kPrepTokens * 2 * G; i += 256) {
        const int tt = i / (2 * G), w = i - tt * 2 * G;
        const float* x = seg_s + tt * seg + (w < G ? w * N : GN + (w - G) * N);
        sc_s[i] = bc_norm_scale_lds(x, N, w < G ? p.b_eps : p.c_eps);
    }
    for (int i = tid; i < kPrepTokens * H; i += 256) {
        const int tt = i / H, h = i - tt * H;
        const float* raw = seg_s + tt * seg + 2 * GN;
        const float dt = softplus_f(raw[h] + p.dt_bias[h]);
        dt_s[i] = dt;
        if (tt < ntok) {
            const float a = -fmaxf(heavy_tail_f(raw[H + h]), p.a_floor);
            const int64_t idx = (tok0 + tt) * H + h;
            step_coefficients(a * dt, dt, raw[2 * H + h], p.alpha + idx, p.beta + idx, p.gamma + idx);
        }
    }
    __syncthreads();
    const int HN = H * N;
    const int heads_per_group = H / G;
    for (int i = tid; i < ntok * HN; i += 256) {
        const int tt = i / HN, rem = i - tt * HN;
        const int h = rem / N, n = rem - h * N;
        const int g = h / heads_per_group;
        const float* x = seg_s + tt * seg;
        const float* sc = sc_s + tt * 2 * G;
        const int64_t o = (tok0 + tt) * HN + rem;
        p.k[o] = (x[g * N + n] * sc[g]) * bw_s[n] + bb_s[rem];
        p.q[o] = (x[GN + g * N + n] * sc[G + g]) * bw_s[N + n] + bb_s[HN + rem];
    }
    const int HR = H * R;
    for (int i = tid; i < ntok * HR; i += 256) {
        const int tt = i / HR, rem = i - tt * HR;
        const int h = rem / R, r = rem - h * R;
        const float* ang = seg_s + tt * seg + 2 * GN + 3 * H;
        p.term[(tok0 + tt) * HR + rem] = (tanhf_cr(ang[r]) * kPiF) * dt_s[tt * H + h];
    }
}

size_t prep_lds_bytes(int tokens_per_block, int64_t N, int64_t G, int64_t H, int64_t R) {
    return sizeof(float) *
           static_cast<size_t>(tokens_per_block * (2 * G * N + 3 * H + R + 2 * G + H) + 2 * N + 2 * H * N);
}

// Phase B + C for one (window, head): the angle terms of a run of tokens are
// staged in LDS, lane r < R carries the fp64 running sum of angle r down the
// run (rounded to fp32 at each token), then every (token, angle) pair is
// wrapped, turned into sin/cos and applied to q and k in parallel.
constexpr int kRotateLds = 4096;

__global__ __launch_bounds__(256) void rotate_kernel(int64_t B, int64_t L, int64_t H, int64_t N, int64_t R,
                                                     const float* __restrict__ term, float* __restrict__ q,
                                                     float* __restrict__ k) {
    __shared__ float cum_s[kRotateLds];
    const int64_t h = blockIdx.x % H;
    const int64_t b = blockIdx.x / H;
    const int tid = threadIdx.x;
    const int Ri = static_cast<int>(R);
    const int run_len = kRotateLds / Ri;
    double running = 0.0;
    for (int64_t t0 = 0; t0 < L; t0 += run_len) {
        const int n = static_cast<int>(L - t0 < run_len ? L - t0 : run_len);
        for (int i = tid; i < n * Ri; i += 256) {
            const int tt = i / Ri, r = i - tt * Ri;
            cum_s[i] = term[((b * L + t0 + tt) * H + h) * R + r];
        }
        __syncthreads();
        if (tid < Ri) {
            for (int tt = 0; tt < n; ++tt) {
                running += static_cast<double>(cum_s[tt * Ri + tid]);
                cum_s[tt * Ri + tid] = static_cast<float>(running);
            }
        }
        __syncthreads();
        for (int i = tid; i < n * Ri; i += 256) {
            const int tt = i / Ri, r = i - tt * Ri;
            const float cumulative = cum_s[i];
            const float wraps = __fmul_rn(kTwoPiF, floorf(cumulative / kTwoPiF));
            double sd, cd;
            sincos_d(static_cast<double>(cumulative - wraps), &sd, &cd);
            const float sine = static_cast<float>(sd);
            const float cosine = static_cast<float>(cd);
            const int64_t th = (b * L + t0 + tt) * H + h;
            float* qp = q + th * N + 2 * r;
            float* kp = k + th * N + 2 * r;
            const float ql = qp[0], qr = qp[1], kl = kp[0], kr = kp[1];
            qp[0] = fmaf(ql, cosine, -(qr * sine));
            qp[1] = fmaf(ql, sine, qr * cosine);
            kp[0] = fmaf(kl, cosine, -(kr * sine));
            kp[1] = fmaf(kl, sine, kr * cosine);
        }
        __syncthreads();
    }
}

struct Strides3 {
    int64_t b, t, h;
};

// Per-token coefficients for mamba3_siso_recurrent (montlok.cpp:279-299).
__global__ __launch_bounds__(256) void coef_kernel(int64_t B, int64_t L, int64_t H, const float* adt, Strides3 as,
                                                   const float* dt, Strides3 ds, const float* trap, Strides3 ts_,
                                                   float* alpha, float* beta, float* gamma) {
    const int idx = static_cast<int>(blockIdx.x * blockDim.x + threadIdx.x);  // B*L*H < 2^31 (checked)
    if (idx >= B * L * H) return;
    const int Hi = static_cast<int>(H), Li = static_cast<int>(L);
    const int bt = idx / Hi, h = idx - bt * Hi;
    const int b = bt / Li, t = bt - b * Li;
    step_coefficients(adt[b * as.b + t * as.t + h * as.h], dt[b * ds.b + t * ds.t + h * ds.h],
                      trap[b * ts_.b + t * ts_.t + h * ts_.h], alpha + idx, beta + idx, gamma + idx);
}

struct RecArgs {
    int64_t B, L, H, N, D;
    const float* q;
    Strides3 qs;
    const float* k;
    Strides3 ks;
    const float* v;
    Strides3 vs;
    const float* gate;
    Strides3 gs;
    int gate_logits;
    const float* alpha;  // [B, L, H] contiguous
    const float* beta;
    const float* gamma;
    const float* skip;   // [H]
    float* out;
    Strides3 os;
};

// The recurrence proper: one wave per (window, head, 64 headdim columns),
// lane = column, state column s[n] in registers, time sequential. q, k, the
// coefficients, v and gate of kStepsPerChunk tokens are staged in LDS
// (double-buffered); the next chunk's global loads are issued before the
// current chunk is computed, so no step waits on memory. NM is the register
// capacity of the state column; EXACT means N == NM.
constexpr int kStepsPerChunk = 8;

template <int NM>
struct RecChunk {
    static constexpr int kTC = kStepsPerChunk;
    static constexpr int kQPL = (kTC * NM + 63) / 64;  // staged q (and k) values per lane
    float q[kQPL], k[kQPL], c, v[kTC], g[kTC];
};

template <int NM, bool EXACT>
__device__ __forceinline__ void rec_fetch(RecChunk<NM>& r, int64_t t0, int64_t L, int N, int lane, bool active,
                                          const float* __restrict__ qrow, int64_t qst,
                                          const float* __restrict__ krow, int64_t kst,
                                          const float* __restrict__ vrow, int64_t vst,
                                          const float* __restrict__ grow, int64_t gst,
                                          const float* __restrict__ alpha, const float* __restrict__ beta,
                                          const float* __restrict__ gamma, int64_t cbase, int64_t H) {
    constexpr int TC = RecChunk<NM>::kTC;
#pragma unroll
    for (int j = 0; j < RecChunk<NM>::kQPL; ++j) {
        const int idx = lane + 64 * j;
        const int tt = idx / NM, n = idx % NM;
        const int64_t t = t0 + tt;
        const bool ok = tt < TC && (EXACT || n < N) && t < L;
        r.q[j] = ok ? qrow[t * qst + n] : 0.0f;
        r.k[j] = ok ? krow[t * kst + n] : 0.0f;
    }
    r.c = 0.0f;
    if (lane < 3 * TC) {
        const int which = lane / TC;
        const int64_t t = t0 + lane % TC;
        const float* src = which == 0 ? alpha : (which == 1 ? beta : gamma);
        if (t < L) r.c = src[cbase + t * H];
    }
#pragma unroll
    for (int tt = 0; tt < TC; ++tt) {
        const int64_t t = t0 + tt;
        const bool ok = active && t < L;
        r.v[tt] = ok ? vrow[t * vst] : 0.0f;
        r.g[tt] = ok ? grow[t * gst] : 0.0f;
    }
}

template <int NM>
__device__ __forceinline__ void rec_commit(const RecChunk<NM>& r, int lane, float* q_s, float* k_s, float* c_s,
                                           float* v_s, float* g_s) {
    constexpr int TC = RecChunk<NM>::kTC;
#pragma unroll
    for (int j = 0; j < RecChunk<NM>::kQPL; ++j) {
        const int idx = lane + 64 * j;
        if (idx < TC * NM) {
            q_s[idx] = r.q[j];
            k_s[idx] = r.k[j];
        }
    }
    if (lane < 3 * TC) c_s[(lane % TC) * 4 + lane / TC] = r.c;
#pragma unroll
    for (int tt = 0; tt < TC; ++tt) {
        v_s[tt * 64 + lane] = r.v[tt];
        g_s[tt * 64 + lane] = r.g[tt];
    }
}

// Lane layout. VEC is the reference's vector path (headdim a multiple of 8)
// with even/odd state-row accumulators (montlok_kernel.h:300-322), y =
// acc_even + acc_odd; otherwise one accumulator. Default: 64 columns per
// wave, one lane per column holding every state row. PAIR (VEC with headdim
// <= 32, where half a wave would idle): 32 columns per wave, two lanes per
// column; the lane of parity p owns the rows n = p (mod 2) and their
// accumulator, and the pair's two sums are added in the reference's order.
template <int NM, bool EXACT, bool VEC, bool PAIR>
__global__ __launch_bounds__(64) void rec_kernel(int64_t L, int64_t H, int64_t D, int N,
                                                 const float* __restrict__ q, Strides3 qs,
                                                 const float* __restrict__ k, Strides3 ks,
                                                 const float* __restrict__ v, Strides3 vs,
                                                 const float* __restrict__ gate, Strides3 gs, int gate_logits,
                                                 const float* __restrict__ alpha, const float* __restrict__ beta,
                                                 const float* __restrict__ gamma, const float* __restrict__ skip_p,
                                                 float* __restrict__ out, Strides3 os) {
    constexpr int TC = kStepsPerChunk;
    constexpr int kCols = PAIR ? 32 : 64;     // columns per wave
    constexpr int kRows = PAIR ? NM / 2 : NM;  // state rows per lane
    __shared__ float q_s[2][TC * NM];
    __shared__ float k_s[2][TC * NM];
    __shared__ float c_s[2][TC * 4];
    __shared__ float v_s[2][TC * 64];
    __shared__ float g_s[2][TC * 64];
    const int64_t blocks_per_head = (D + kCols - 1) / kCols;
    const int64_t item = blockIdx.x;
    const int64_t dblk = item % blocks_per_head;
    const int64_t bh = item / blocks_per_head;
    const int64_t h = bh % H;
    const int64_t b = bh / H;
    const int lane = threadIdx.x;
    const int par = PAIR ? lane >> 5 : 0;
    const int64_t d = dblk * kCols + (PAIR ? (lane & 31) : lane);
    const bool active = d < D;
    if (EXACT) N = NM;

    float s[kRows];
#pragma unroll
    for (int m = 0; m < kRows; ++m) s[m] = 0.0f;
    const float skip = skip_p[h];
    const float* qrow = q + b * qs.b + h * qs.h;
    const float* krow = k + b * ks.b + h * ks.h;
    const float* vrow = v + b * vs.b + h * vs.h + (active ? d : 0);
    const float* grow = gate + b * gs.b + h * gs.h + (active ? d : 0);
    float* orow = out + b * os.b + h * os.h + (active ? d : 0);
    const int64_t cbase = b * L * H + h;

    RecChunk<NM> pre;
    rec_fetch<NM, EXACT>(pre, 0, L, N, lane, active, qrow, qs.t, krow, ks.t, vrow, vs.t, grow, gs.t, alpha, beta,
                         gamma, cbase, H);
    rec_commit<NM>(pre, lane, q_s[0], k_s[0], c_s[0], v_s[0], g_s[0]);
    __syncthreads();
    float v_last = 0.0f;
    for (int64_t t0 = 0, c = 0; t0 < L; t0 += TC, ++c) {
        const int buf = static_cast<int>(c & 1);
        const bool more = t0 + TC < L;
        if (more) {
            rec_fetch<NM, EXACT>(pre, t0 + TC, L, N, lane, active, qrow, qs.t, krow, ks.t, vrow, vs.t, grow, gs.t,
                                 alpha, beta, gamma, cbase, H);
        }
        const int steps = static_cast<int>(more ? TC : L - t0);
#pragma unroll 1
        for (int tt = 0; tt < steps; ++tt) {
            const int64_t t = t0 + tt;
            const float al = c_s[buf][tt * 4], be = c_s[buf][tt * 4 + 1], ga = c_s[buf][tt * 4 + 2];
            const float* qt = &q_s[buf][tt * NM];
            const float* kt = &k_s[buf][tt * NM];
            const float* kp = tt > 0 ? &k_s[buf][(tt - 1) * NM] : (t > 0 ? &k_s[buf ^ 1][(TC - 1) * NM] : kt);
            const float v_cur = v_s[buf][tt * 64 + lane];
            const float v_prev = tt > 0 ? v_s[buf][(tt - 1) * 64 + lane] : v_last;
            const float g_cur = g_s[buf][tt * 64 + lane];
            const float pv = t > 0 ? be * v_prev : 0.0f;
            const float cv = ga * v_cur;
            float acc0 = 0.0f, acc1 = 0.0f;
#pragma unroll
            for (int m = 0; m < kRows; ++m) {
                const int n = PAIR ? 2 * m + par : m;
                if (EXACT || n < N) {
                    float upd;
                    if (VEC || t > 0) {
                        upd = fmaf(kt[n], cv, fmaf(s[m], al, kp[n] * pv));
                    } else {
                        upd = fmaf(kt[n], cv, s[m] * al);
                    }
                    s[m] = upd;
                    if (!PAIR && VEC && (n & 1)) {
                        acc1 = fmaf(upd, qt[n], acc1);
                    } else {
                        acc0 = fmaf(upd, qt[n], acc0);
                    }
                }
            }
            float sum;
            if constexpr (PAIR) {
                const float other = __shfl_xor(acc0, 32);
                sum = par == 0 ? acc0 + other : other + acc0;  // acc_even + acc_odd
            } else {
                sum = VEC ? acc0 + acc1 : acc0;
            }
            const float y = fmaf(skip, v_cur, sum);
            float o;
            if (gate_logits) {
                const double z = static_cast<double>(g_cur);
                o = static_cast<float>(static_cast<double>(y) * silu_d(z));
            } else {
                o = y * g_cur;
            }
            if (active && par == 0) orow[t * os.t] = o;
        }
        if (more) {
            // The chunk before this one (buffer buf ^ 1) was last read at tt = 0 above.
            v_last = v_s[buf][(TC - 1) * 64 + lane];
            __syncthreads();
            rec_commit<NM>(pre, lane, q_s[buf ^ 1], k_s[buf ^ 1], c_s[buf ^ 1], v_s[buf ^ 1], g_s[buf ^ 1]);
            __syncthreads();
        }
    }
}

// ---------------------------------------------------------------------------
// The recurrence in chunked form, on the fp32 matrix cores
// ---------------------------------------------------------------------------
//
// Over a chunk of C tokens (chunk-local indices t, s in [0, C)), unrolling
// S_t = a_t S_{t-1} + b_t k_{t-1} v_{t-1}^T + g_t k_t v_t^T gives
//   y_t = sum_{s<=t} W[t][s] (q_t . k_s) v_s          intra-chunk
//       + Din(t) S_in^T q_t                            carried state
//       + Wp(t) (q_t . k_p) v_p                        the previous chunk's last token p
//   W[t][s] = g_s prod_{r=s+1..t} a_r + [s < t] b_{s+1} prod_{r=s+2..t} a_r
//   Din(t)  = prod_{r=0..t} a_r,  Wp(t) = b_0 prod_{r=1..t} a_r
// and the state after the chunk is
//   S_out = Din(C-1) S_in + sum_s W[C-1][s] k_s v_s^T + Wp(C-1) k_p v_p^T.
// The products of the stored fp32 coefficients are formed in double, one lane
// per s walking t forward (no exp or log: exactly the products the
// time-sequential form multiplies by), and each weight is rounded to fp32
// once. One wave per (window, head), all D <= 64 columns:
//   G^T = K Q^T        v_mfma_f32_16x16x4_f32, A = K rows, B = Q rows (float4
//                      loads: instruction v of a 16-wide k block takes
//                      k = 4g + v in lane group g on both sides);
//   P = W o G          the accumulator layout of G^T (s = 4g + v, t = lane % 16)
//                      is the A-operand layout of P for Y = P V;
//   Y = P V + Q S_in   V staged in LDS; S_in lives in registers in the
//                      accumulator layout (n = 4g + v, d = lane % 16), which is
//                      the B-operand layout of Q S_in and the C operand of the
//                      state update S_out = Din S_in + K^T (w o V).
// Every fp32 sum is in an order of its own, so results agree with the
// time-sequential kernel to rounding (the fp32 tolerance), not bit for bit.
typedef float f32x4_t __attribute__((ext_vector_type(4)));

template <int C, int NT, int DT>
__global__ __launch_bounds__(64) void rec_chunk_kernel(RecArgs a) {
    constexpr int N = 16 * NT, D = 16 * DT;
    constexpr int CT = C / 16;
    constexpr int WP = C + 4;  // row pitches in floats: 16-byte rows, 16 consecutive rows on distinct banks
    constexpr int NP = N + 4;
    constexpr int VP = D + 4;
    __shared__ __attribute__((aligned(16))) float w_s[C * WP];
    __shared__ __attribute__((aligned(16))) float q_sh[C * NP];
    __shared__ __attribute__((aligned(16))) float k_sh[C * NP];
    __shared__ __attribute__((aligned(16))) float v_sh[C * VP];
    __shared__ __attribute__((aligned(16))) float g_sh[C * VP];
    __shared__ float coef[3][C];
    __shared__ float din_s[C], wp_s[C], ck_s[C];
    __shared__ float kp_s[N];

    const int lane = threadIdx.x, g = lane >> 4, li = lane & 15;
    const int64_t L = a.L, H = a.H;
    const int64_t h = blockIdx.x % H, b = blockIdx.x / H;
    const float* qrow = a.q + b * a.qs.b + h * a.qs.h;
    const float* krow = a.k + b * a.ks.b + h * a.ks.h;
    const float* vrow = a.v + b * a.vs.b + h * a.vs.h;
    const float* grow = a.gate + b * a.gs.b + h * a.gs.h;
    float* orow = a.out + b * a.os.b + h * a.os.h;
    const int64_t cbase = b * L * H + h;
    const float skip = a.skip[h];

    f32x4_t S[NT][DT];
    float vp_d[DT];
#pragma unroll
    for (int nt = 0; nt < NT; ++nt)
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) S[nt][dt] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) vp_d[dt] = 0.0f;

    for (int64_t c0 = 0; c0 < L; c0 += C) {
        const int Lc = static_cast<int>(L - c0 < C ? L - c0 : C);
        const bool first = c0 == 0, last = c0 + C >= L;
        // 1. The chunk's operands into LDS, every load of a batch issued before
        //    the first wait (rows past the end read the last row; their
        //    coefficients are zero, so they carry no weight).
        {
            constexpr int QU = C * N / 4 / 64;  // float4 units of Q (and K) per lane
            float4 qq[QU], kk[QU];
            constexpr int CU = (3 * C + 63) / 64;  // coefficient entries (alpha, beta, gamma of C tokens) per lane
            float cf[CU];
#pragma unroll
            for (int j = 0; j < QU; ++j) {
                const int u = lane + 64 * j, s = u / (N / 4), n4 = 4 * (u % (N / 4));
                const int64_t t = c0 + (s < Lc ? s : Lc - 1);
                qq[j] = *reinterpret_cast<const float4*>(qrow + t * a.qs.t + n4);
                kk[j] = *reinterpret_cast<const float4*>(krow + t * a.ks.t + n4);
            }
#pragma unroll
            for (int j = 0; j < CU; ++j) {
                const int u = lane + 64 * j, which = u / C, s = u % C;
                const float* src = which == 0 ? a.alpha : (which == 1 ? a.beta : a.gamma);
                cf[j] = u < 3 * C && s < Lc ? src[cbase + (c0 + s) * H] : 0.0f;
            }
#pragma unroll
            for (int j = 0; j < QU; ++j) {
                const int u = lane + 64 * j, s = u / (N / 4), n4 = 4 * (u % (N / 4));
                *reinterpret_cast<float4*>(q_sh + s * NP + n4) = qq[j];
                *reinterpret_cast<float4*>(k_sh + s * NP + n4) = kk[j];
            }
#pragma unroll
            for (int j = 0; j < CU; ++j) {
                const int u = lane + 64 * j;
                if (u < 3 * C) coef[u / C][u % C] = cf[j];
            }
            constexpr int VU = C * D / 64;
            float vv[VU], gg[VU];
#pragma unroll
            for (int j = 0; j < VU; ++j) {
                const int u = lane + 64 * j, s = u / D, d = u % D;
                const int64_t t = c0 + (s < Lc ? s : Lc - 1);
                vv[j] = vrow[t * a.vs.t + d];
                gg[j] = grow[t * a.gs.t + d];
            }
#pragma unroll
            for (int j = 0; j < VU; ++j) {
                const int u = lane + 64 * j;
                v_sh[(u / D) * VP + u % D] = vv[j];
                g_sh[(u / D) * VP + u % D] = gg[j];
            }
        }
        __syncthreads();
        // 2. Weights: lane s walks t forward; lane 0 also writes Din and Wp.
        if (lane < C) {
            const int s = lane;
            const double gam = coef[2][s];
            const double bet = s + 1 < C ? static_cast<double>(coef[1][s + 1]) : 0.0;
            const double a0 = coef[0][0], b0 = first ? 0.0 : static_cast<double>(coef[1][0]);
            double d = 1.0, e = 1.0;
#pragma unroll
            for (int t = 0; t < C; ++t) {
                float w = 0.0f;
                const double at = coef[0][t];
                if (t >= s) {
                    if (t > s) d *= at;
                    if (t > s + 1) e *= at;
                    double val = gam * d;
                    if (t > s) val = fma(bet, e, val);
                    w = static_cast<float>(val);
                }
                w_s[t * WP + s] = w;
                if (s == 0) {
                    din_s[t] = static_cast<float>(a0 * d);
                    wp_s[t] = static_cast<float>(b0 * d);
                }
            }
            // 3. The previous chunk's last token: ck[t] = Wp(t) (q_t . k_p), computed by lane t.
            float dot = 0.0f;
            if (!first) {
#pragma unroll
                for (int n = 0; n < N; ++n) dot = fmaf(q_sh[s * NP + n], kp_s[n], dot);
            }
            ck_s[s] = dot;
        }
        __syncthreads();
        if (lane < C) ck_s[lane] *= wp_s[lane];
        __syncthreads();

        // 4. Outputs, 16 tokens at a time; every operand from LDS. Independent
        //    accumulators (the s tiles of G, the d tiles of Y) are interleaved so
        //    that consecutive MFMAs do not wait on each other.
#pragma unroll
        for (int tt = 0; tt < CT; ++tt) {
            const int t0 = 16 * tt;
            if (t0 >= Lc) break;
            float4 qf[NT];
#pragma unroll
            for (int nt = 0; nt < NT; ++nt) qf[nt] = *reinterpret_cast<const float4*>(q_sh + (t0 + li) * NP + 16 * nt + 4 * g);
            f32x4_t P[CT];
#pragma unroll
            for (int st = 0; st < CT; ++st) P[st] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int nt = 0; nt < NT; ++nt) {
                float4 k4[CT];
#pragma unroll
                for (int st = 0; st < CT; ++st) {
                    if (st <= tt) k4[st] = *reinterpret_cast<const float4*>(k_sh + (16 * st + li) * NP + 16 * nt + 4 * g);
                }
#pragma unroll
                for (int st = 0; st < CT; ++st) {
                    if (st > tt) continue;
                    P[st] = __builtin_amdgcn_mfma_f32_16x16x4f32(k4[st].x, qf[nt].x, P[st], 0, 0, 0);
                }
#pragma unroll
                for (int st = 0; st < CT; ++st) {
                    if (st > tt) continue;
                    P[st] = __builtin_amdgcn_mfma_f32_16x16x4f32(k4[st].y, qf[nt].y, P[st], 0, 0, 0);
                }
#pragma unroll
                for (int st = 0; st < CT; ++st) {
                    if (st > tt) continue;
                    P[st] = __builtin_amdgcn_mfma_f32_16x16x4f32(k4[st].z, qf[nt].z, P[st], 0, 0, 0);
                }
#pragma unroll
                for (int st = 0; st < CT; ++st) {
                    if (st > tt) continue;
                    P[st] = __builtin_amdgcn_mfma_f32_16x16x4f32(k4[st].w, qf[nt].w, P[st], 0, 0, 0);
                }
            }
#pragma unroll
            for (int st = 0; st < CT; ++st) {  // P = W o G
                if (st > tt) continue;
                const float4 w4 = *reinterpret_cast<const float4*>(w_s + (t0 + li) * WP + 16 * st + 4 * g);
                P[st] = f32x4_t{w4.x * P[st][0], w4.y * P[st][1], w4.z * P[st][2], w4.w * P[st][3]};
            }
            f32x4_t Y[DT], Yi[DT];
#pragma unroll
            for (int dt = 0; dt < DT; ++dt) {
                Y[dt] = f32x4_t{0.f, 0.f, 0.f, 0.f};
                Yi[dt] = f32x4_t{0.f, 0.f, 0.f, 0.f};
            }
#pragma unroll
            for (int st = 0; st < CT; ++st) {
                if (st > tt) continue;
#pragma unroll
                for (int v = 0; v < 4; ++v) {
                    float vb[DT];
#pragma unroll
                    for (int dt = 0; dt < DT; ++dt) vb[dt] = v_sh[(16 * st + 4 * g + v) * VP + 16 * dt + li];
#pragma unroll
                    for (int dt = 0; dt < DT; ++dt) Y[dt] = __builtin_amdgcn_mfma_f32_16x16x4f32(P[st][v], vb[dt], Y[dt], 0, 0, 0);
                }
            }
            if (!first) {
#pragma unroll
                for (int nt = 0; nt < NT; ++nt) {
                    const float qv[4] = {qf[nt].x, qf[nt].y, qf[nt].z, qf[nt].w};
#pragma unroll
                    for (int v = 0; v < 4; ++v) {
#pragma unroll
                        for (int dt = 0; dt < DT; ++dt) {
                            Yi[dt] = __builtin_amdgcn_mfma_f32_16x16x4f32(qv[v], S[nt][dt][v], Yi[dt], 0, 0, 0);
                        }
                    }
                }
            }
#pragma unroll
            for (int dt = 0; dt < DT; ++dt) {
                const int d = 16 * dt + li;
#pragma unroll
                for (int v = 0; v < 4; ++v) {
                    const int t = t0 + 4 * g + v;
                    if (t >= Lc) continue;
                    float y = Y[dt][v];
                    if (!first) y = fmaf(ck_s[t], vp_d[dt], fmaf(din_s[t], Yi[dt][v], y));
                    y = fmaf(skip, v_sh[t * VP + d], y);
                    const float gt = g_sh[t * VP + d];
                    float o;
                    if (a.gate_logits) {
                        const double z = static_cast<double>(gt);
                        o = static_cast<float>(static_cast<double>(y) * silu_d(z));
                    } else {
                        o = y * gt;
                    }
                    orow[(c0 + t) * a.os.t + d] = o;
                }
            }
        }
        if (last) break;

        // 5. State after the chunk (every token of a non-final chunk is valid);
        //    the NT x DT state tiles are independent accumulators, interleaved.
        {
            const float dl = din_s[C - 1], wl = wp_s[C - 1];
#pragma unroll
            for (int nt = 0; nt < NT; ++nt)
#pragma unroll
                for (int dt = 0; dt < DT; ++dt)
#pragma unroll
                    for (int v = 0; v < 4; ++v) {
                        float x = S[nt][dt][v] * dl;
                        if (!first) x = fmaf(wl * kp_s[16 * nt + 4 * g + v], vp_d[dt], x);
                        S[nt][dt][v] = x;
                    }
#pragma unroll
            for (int st = 0; st < CT; ++st) {
#pragma unroll
                for (int v = 0; v < 4; ++v) {
                    const int srow = 16 * st + 4 * g + v;
                    const float wv = w_s[(C - 1) * WP + srow];
                    float kA[NT], bv[DT];
#pragma unroll
                    for (int nt = 0; nt < NT; ++nt) kA[nt] = k_sh[srow * NP + 16 * nt + li];
#pragma unroll
                    for (int dt = 0; dt < DT; ++dt) bv[dt] = wv * v_sh[srow * VP + 16 * dt + li];
#pragma unroll
                    for (int nt = 0; nt < NT; ++nt)
#pragma unroll
                        for (int dt = 0; dt < DT; ++dt)
                            S[nt][dt] = __builtin_amdgcn_mfma_f32_16x16x4f32(kA[nt], bv[dt], S[nt][dt], 0, 0, 0);
                }
            }
        }
        __syncthreads();  // kp_s and this chunk's LDS operands are read above
        if (lane < N) kp_s[lane] = k_sh[(C - 1) * NP + lane];
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) vp_d[dt] = v_sh[(C - 1) * VP + 16 * dt + li];
        __syncthreads();
    }
}

// ---------------------------------------------------------------------------
// The whole forward in one kernel: in_proj post-processing + chunked scan
// ---------------------------------------------------------------------------
//
// One block of DT waves per (window, head); wave w owns headdim columns
// [16w, 16w + 16). Per 32-token chunk, straight from the in_proj rows:
//   a. the head's B and C group rows, its dt/A/trap logits and the angles into
//      LDS; this wave's v (x) and gate (z) columns into registers, laid out as
//      the operands below take them (token 16st + 4g + v, column 16w + li);
//   b. the BCNorm scales (one lane per token and group), (alpha, beta, gamma,
//      dt) per token, tanh(angle) * pi;
//   c. q and k (scale, norm weight, bias) in place; the fp64 running angle
//      sums (one lane per angle, carried across chunks in a register); the
//      decay weights W, Din, Wp;
//   d. the rotation of each (2r, 2r + 1) pair of q and k;
//   e. the G^T = K Q^T tiles, one wave per tile, masked by W into LDS; the
//      previous chunk's last-token term ck;
//   f. each wave's output columns, Y = P V + Din Q S_in + ck v_p, skip, gate;
//   g. each wave's state columns, S_out = Din S_in + Wp k_p v_p^T + K^T (w o V).
// Steps a-d are prep_kernel's and rotate_kernel's arithmetic per token, and
// e-g rec_chunk_kernel's products in the same order, so the output equals the
// prep -> rotate -> rec_chunk_kernel sequence bit for bit; q and k never leave
// LDS. Blocks are ordered so that the heads of one window run on one XCD and
// share its L2 copy of the window's B/C rows.
// sin and cos of a running angle sum, reduced by whole turns in fp32 first.
__device__ __forceinline__ void rotation_of(float cumulative, float* sine, float* cosine) {
    const float wraps = __fmul_rn(kTwoPiF, floorf(cumulative / kTwoPiF));
    double sd, cd;
    sincos_d(static_cast<double>(cumulative - wraps), &sd, &cd);
    *sine = static_cast<float>(sd);
    *cosine = static_cast<float>(cd);
}

// The step coefficients of token ct < C of a chunk (one lane per token):
// dt = softplus(dt logit + bias), A = -max(heavy_tail(A logit), floor), then
// (alpha, beta, gamma) by step_coefficients (zero for tokens past Lc) and dt.
template <int C>
__device__ __forceinline__ void token_coefficients(int ct, float dt_logit, float a_logit, float trap_logit,
                                                   float dt_bias, float a_floor, int Lc, float (&coef)[4][C]) {
    const float dt = softplus_f(dt_logit + dt_bias);
    const float am = -fmaxf(heavy_tail_f(a_logit), a_floor);
    float al, be, ga;
    step_coefficients(am * dt, dt, trap_logit, &al, &be, &ga);
    const bool valid = ct < Lc;
    coef[0][ct] = valid ? al : 0.0f;
    coef[1][ct] = valid ? be : 0.0f;
    coef[2][ct] = valid ? ga : 0.0f;
    coef[3][ct] = dt;
}

// The decay weights of one chunk into w_s (rows of C + 4; column C holds
// Din, C + 1 Wp; row C is a sink), walked by lane ct (0 .. 63) of one wave
// that sees the chunk's coefficients. Lane s < C walks t = s + 1, s + 2, ...
// (lanes drop out past the chunk end), carrying the products
// prod_{s<r<=t} alpha_r and prod_{s+1<r<=t} alpha_r in fp64; its alpha values
// are read 8 steps ahead. W[t][s] for t < s is never read (the G tiles mask
// it). Lanes C and C + 1 write Din(t) = a_0 prod_{0<r<=t} a_r and
// Wp(t) = b_0 prod_{0<r<=t} a_r as the weights of a column s = 0 with
// gamma = a_0 (b_0) and no beta term (b_0 = 0 in the first chunk).
template <int C, bool kSplit>
__device__ __forceinline__ void decay_walk(int ct, bool first, const float (&coef)[4][C], float* w_s) {
    constexpr int WP = C + 4, kDin = C, kWp = C + 1;
    // Walkers: columns s < C, then Din (column kDin) and Wp (kWp), both
    // with s = 0. Lane w < C + 2 walks t = s + 1 .. s + 16 of walker
    // w; a walk longer than 16 steps (s < C - 17, and Din, Wp) has a
    // second lane, C + 2 + j, for t = s + 17 .. C - 1. That lane first
    // runs 16 multiply-only steps to form the same sequential
    // products the first lane holds at t = s + 16, so every weight is
    // bit-identical to one lane walking the whole column, while the
    // wave issues 16 full steps instead of 31. Four-wave blocks keep
    // one lane per walker (32 full steps): the split's registers cost
    // them more than the shorter walk saves.
    constexpr int kFull = kSplit ? 16 : 32;  // full steps per lane (whole batches of 8)
    constexpr int kLong = C - 17;  // columns whose walk exceeds 16 steps
    static_assert(C + 2 + kLong + 2 <= 64, "the walkers' lanes must fit one wave");
    const int hf = kSplit && ct >= C + 2 ? 1 : 0;
    const int j2 = ct - (C + 2);
    const int wl = hf == 0 ? ct : (j2 < kLong ? j2 : C + (j2 - kLong));
    if (ct >= 0 && (hf == 0 ? ct < C + 2 : j2 < kLong + 2)) {
        const int s = wl < C ? wl : 0;
        const double b0 = first ? 0.0 : static_cast<double>(coef[1][0]);
        const double gam = wl < C ? static_cast<double>(coef[2][s]) : (wl == C ? static_cast<double>(coef[0][0]) : b0);
        const double bet = wl + 1 < C ? static_cast<double>(coef[1][wl + 1]) : 0.0;
        const int colw = wl < C ? wl : (wl == C ? kDin : kWp);
        if (hf == 0) w_s[s * WP + colw] = static_cast<float>(gam * 1.0);  // t = s
        // Step k handles t = s + 1 + k with alpha from a clamped slot;
        // steps with t >= C store into the sink row C, so no step is
        // predicated.
        double dd = 1.0, e = 1.0;
        if constexpr (kSplit) {
            float al[16];
#pragma unroll
            for (int k = 0; k < 16; ++k) al[k] = coef[0][min(s + 1 + k, C - 1)];
#pragma unroll
            for (int k = 0; k < 16; ++k) {
                const double at = al[k];
                dd *= at;
                if (k > 0) e *= at;
            }
        }
        if (hf == 0) {  // (the first lane walks from t = s + 1)
            dd = 1.0;
            e = 1.0;
        }
        const int kb = 16 * hf;
        float nx[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) nx[i] = coef[0][min(s + 1 + kb + i, C - 1)];
        auto batch = [&](int k0) {  // steps k0 .. k0 + 7, the next batch's alpha values read ahead
            float al[8];
#pragma unroll
            for (int i = 0; i < 8; ++i) al[i] = nx[i];
            if (k0 + 8 < kFull) {
#pragma unroll
                for (int i = 0; i < 8; ++i) nx[i] = coef[0][min(s + 1 + kb + k0 + 8 + i, C - 1)];
            }
            // Each group of 4 steps runs the two product chains first,
            // then the 4 independent weights, then the 4 stores.
#pragma unroll
            for (int i0 = 0; i0 < 8; i0 += 4) {
                double ddv[4], ev[4];
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const double at = al[i0 + i];
                    dd *= at;
                    if (kb + k0 + i0 + i > 0) e *= at;
                    ddv[i] = dd;
                    ev[i] = e;
                }
                float wv[4];
#pragma unroll
                for (int i = 0; i < 4; ++i) wv[i] = static_cast<float>(fma(bet, ev[i], gam * ddv[i]));
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const int t = s + 1 + kb + k0 + i0 + i;
                    w_s[(t < C ? t : C) * WP + colw] = wv[i];
                }
            }
        };
        // The split walk's two batches are straight-line code; the one-lane walk (32 steps) keeps
        // a loop, whose registers the four-wave blocks cannot spare unrolled.
        if constexpr (kSplit) {
            batch(0);
            batch(8);
        } else {
#pragma unroll 1
            for (int k0 = 0; k0 < kFull; k0 += 8) batch(k0);
        }
    }
}

struct ScanArgs {
    const float* proj;  // [B, L, W] rows: [z | x | B | C | dt | A | trap | angles]
    int64_t sb, st;
    int64_t B, L, G, H, R;
    const float* b_bias;  // [H, N]
    const float* c_bias;
    const float* b_norm_w;  // [N]
    const float* c_norm_w;
    float b_eps, c_eps;
    const float* dt_bias;  // [H]
    float a_floor;
    const float* skip;  // [H]
    const float* gate;  // z columns of proj (gate_logits), or an explicit gate [B, L, H*D]
    int64_t gsb, gst;
    int gate_logits;
    float* out;  // [B, L, H*D] contiguous
};

// The LDS of one (window, head) scan.
template <int C, int NT, int DT>
struct ScanLds {
    static constexpr int N = 16 * NT, CT = C / 16, NP = N + 4, WP = C + 4, NPAIR = CT * (CT + 1) / 2, RM = N / 2;
    __attribute__((aligned(16))) float q_sh[C * NP];
    __attribute__((aligned(16))) float k_sh[C * NP];
    __attribute__((aligned(16))) float w_s[(C + 1) * WP];  // row C: sink of the walk's steps past the chunk
    f32x4_t p_s[NPAIR * 64];
    float ang_s[C * RM];  // angle logits, then tanh(angle) * pi
    float cum_s[C * RM];  // cumulative angles
    float raw_s[3][C];    // dt, A, trap logits
    __attribute__((aligned(16))) float coef[4][C];  // alpha, beta, gamma, dt
    float sc_s[2][C];     // B and C norm scales
    float ck_s[C];
    float kp_s[2][N];
    float nrm_s[4][N];    // B norm weight, C norm weight, this head's B bias, C bias
};

// Called by every thread of the block around each chunk of the scan.
// PREP's split of the outputs: a scan wave forms token tile 0's outputs of its
// columns; the block's other waves form tile 1's. The scan wave also forms the
// tile-1 gates of v < kPrepOwnV (token 16 + 4 g + v) and hands them over at
// hooks.share_gate(v, gate) before the barrier that ends step d.
constexpr int kPrepOwnV = 2;

struct NoChunkHooks {
    __device__ void before(int64_t) const {}
    __device__ void after(int64_t, bool) const {}
    __device__ const float* rotations() const { return nullptr; }
};

// The scan of one (window, head) by the DT waves of threads tid_base ..
// tid_base + 64 DT - 1 of the block, with LDS `sh`. TILE = false: the in_proj
// rows of window b are in global memory at a.proj + b a.sb + t a.st. TILE =
// true: the rows of the current chunk only are at a.proj + (t - c0) a.st
// (LDS, refilled by hooks.before; b and a.sb unused). TILE_OUT (TILE unless
// given) likewise for the outputs: a.out [B, L, d_inner], or the current
// chunk's rows at a.out + (t - c0) d_inner.
// Every thread of the block runs the same sequence of barriers, so several
// heads can share a block. PREP (TILE, one chunk, the first and last; two
// waves; the gate columns in the projection rows, a.gst = a.st): other waves of the block have already formed the chunk's
// coefficients and tanh(angle) * pi (before the barrier that ends
// hooks.before); they form its decay weights before the barrier that ends
// step d, and the running angle sums and the sin/cos of each (token, angle)
// pair at hooks.rotations() ([C][N / 2] pairs) before hooks.wait_rotations()
// returns. Step a skips the dt/A/trap and angle columns; steps a to d run
// without a barrier: each wave forms the norm scales of the rows it scales
// in step c (read from the B/C rows where hooks.before left them) and its
// gates, and rotates those rows in step d; step c skips the angle sums. Steps
// e and f form token tile 0's G tile, products and outputs in registers (tile
// 1's are the other waves' after the barrier that ends step d).
template <int C, int NT, int DT, bool TILE, class Hooks, bool TILE_OUT = TILE, bool PREP = false>
__device__ __forceinline__ void scan_head(const ScanArgs& a, ScanLds<C, NT, DT>& sh, int64_t b, int64_t h,
                                          int tid_base, const Hooks& hooks) {
    static_assert(C == 32, "the BCNorm step takes one lane per (token, B|C) pair of a 64-lane wave");
    static_assert(!PREP || (TILE && DT == 2), "PREP: the tiled two-wave scan");
    static_assert(!PREP || NT == 1, "PREP: step c's rows of a wave are 4 wave + q + 8 j (N = 16, 128 threads)");
    constexpr int N = 16 * NT, D = 16 * DT, NTH = 64 * DT;
    constexpr int CT = C / 16;
    constexpr int NP = N + 4, WP = C + 4;
    constexpr int NPAIR = CT * (CT + 1) / 2;
    constexpr int CTE = PREP ? 1 : CT;  // token tiles whose outputs this scan forms
    constexpr int RM = N / 2;  // rotary angles at most
    constexpr bool kEarlyGate = DT == 2;
    static_assert(NTH % N == 0, "a thread keeps one q/k column across the chunk");
    float* q_sh = sh.q_sh;
    float* k_sh = sh.k_sh;
    float* w_s = sh.w_s;
    f32x4_t* p_s = sh.p_s;
    float* ang_s = sh.ang_s;
    float* cum_s = sh.cum_s;
    auto& raw_s = sh.raw_s;
    auto& coef = sh.coef;
    auto& sc_s = sh.sc_s;
    float* ck_s = sh.ck_s;
    auto& kp_s = sh.kp_s;
    auto& nrm_s = sh.nrm_s;
    // Din(t) and Wp(t) live in the padding columns C and C + 1 of the W rows.
    constexpr int kDin = C, kWp = C + 1;
    static_assert(NPAIR == ScanLds<C, NT, DT>::NPAIR && NP == ScanLds<C, NT, DT>::NP, "LDS layout");

    const int64_t H = a.H, L = a.L, G = a.G;
    const int R = static_cast<int>(a.R);
    const unsigned Hu = static_cast<unsigned>(a.H);
    const int64_t d_inner = H * D, GN = G * N;
    const float* base = TILE ? a.proj : a.proj + b * a.sb;
    const float* brow = base + 2 * d_inner + static_cast<int64_t>(static_cast<unsigned>(h) / (Hu / static_cast<unsigned>(a.G))) * N;
    const float* crow = brow + GN;
    const float* mrow = base + 2 * d_inner + 2 * GN + h;  // dt; A at +H, trap at +2H
    const float* arow = base + 2 * d_inner + 2 * GN + 3 * H;
    const float* xrow = base + d_inner + h * D;
    const float* zrow = (TILE ? a.gate : a.gate + b * a.gsb) + h * D;
    float* orow = (TILE_OUT ? a.out : a.out + b * L * d_inner) + h * D;
    const float skip = a.skip[h], dt_bias = a.dt_bias[h];

    for (int i = static_cast<int>(threadIdx.x) - tid_base; i < N; i += NTH) {
        kp_s[0][i] = 0.0f;  // k_p before the first chunk
        nrm_s[0][i] = a.b_norm_w[i];
        nrm_s[1][i] = a.c_norm_w[i];
        nrm_s[2][i] = a.b_bias[h * N + i];
        nrm_s[3][i] = a.c_bias[h * N + i];
    }
    // (token, angle) work items i < C * R map to t = i / R by a multiply-shift,
    // exact for i < 2^10 and R <= 32.
    const unsigned rmagic = R > 0 ? (65536u + static_cast<unsigned>(R) - 1u) / static_cast<unsigned>(R) : 0u;

    f32x4_t S[NT];  // S[16nt + 4g + v][col]
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) S[nt] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    float vp = 0.0f;        // v of the previous chunk's last token, this lane's column
    double running = 0.0;   // lane r < R: the running angle sum
    float vx[CT][4], zx[CT][4];

    // One chunk; `last` is compile-time, so a full chunk runs without the edge
    // conditions (no partial tiles) and its products and gate arithmetic form
    // long straight-line blocks the scheduler can interleave. The first chunk
    // runs the same code: its carried state, k_p and v_p are zero, so the terms
    // they enter are exact zeros, and a select keeps its outputs those of a
    // scan with no carried state.
    auto chunk = [&](auto last_c, int64_t c0) {
        constexpr bool last = decltype(last_c)::value;
        const bool first = PREP || c0 == 0;  // PREP runs one chunk: known here, so its first-chunk zeros fold
        // The thread index is made opaque per chunk so that the per-lane index
        // arithmetic of the phases below is recomputed here (a few integer
        // operations) rather than hoisted out of the loop and held in VGPRs.
        int tid = static_cast<int>(threadIdx.x) - tid_base;
        asm volatile("" : "+v"(tid));
        const int lane = tid & 63, g = lane >> 4, li = lane & 15;
        const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
        const int col = 16 * wave + li, n_own = tid % N;
        const int Lc = last ? static_cast<int>(L - c0) : C;
        const int par = static_cast<int>((c0 / C) & 1);
        // Output gates of this lane's (token, column) pairs from z alone:
        // silu(z) in double (or z itself for an explicit gate). Two-wave blocks
        // form them in the phases where the wave would otherwise wait (wave 0
        // beside the coefficient wave in b, wave 1 beside the angle sums in c);
        // other blocks just before the outputs. The values are held where they
        // are formed: left to itself the compiler sinks each gate into the
        // predicated store of its output (the last chunk's stores are guarded),
        // where the fp64 chains run one after another.
        double gz[CT][4];
        // PREP: the wave forms the gates of (token tile, v) pairs own(tt, v); the others arrive from
        // the other waves at hooks.late_gates() by the end of step d.
        auto own = [](int tt, int v) { return !PREP || tt == 0 || v < kPrepOwnV; };
        auto gates = [&]() {
#pragma unroll
            for (int tt = 0; tt < CT; ++tt)
#pragma unroll
                for (int v = 0; v < 4; ++v) {
                    if (!own(tt, v)) continue;
                    const double z = static_cast<double>(zx[tt][v]);
                    const double sz = silu_d(z);
                    gz[tt][v] = a.gate_logits ? sz : z;
                }
#pragma unroll
            for (int tt = 0; tt < CT; ++tt)
#pragma unroll
                for (int v = 0; v < 4; ++v)
                    if (own(tt, v)) asm volatile("" : "+v"(gz[tt][v]));
        };
        // a. Every global load of the chunk issued before the first wait
        //    (tokens past the end read the last token; they carry no weight).
        //    Offsets are 32-bit from the chunk's first row (row strides below 2^25 floats, checked at
        //    launch).
        //    PREP reads the tile's rows unclamped: its rows past the end hold
        //    the last token's values already (hooks.before clamps its x rows),
        //    and keeps this thread's B/C values in bx/cx for step c.
        constexpr int BU = C * N / NTH;
        float bx[BU], cx[BU];
        {
            constexpr int MU = (3 * C + NTH - 1) / NTH;
            constexpr int AU = (C * RM + NTH - 1) / NTH;
            const int st32 = static_cast<int>(a.st), gst32 = static_cast<int>(a.gst);
            const int64_t cr = TILE ? 0 : c0 * a.st, cg = TILE ? 0 : c0 * a.gst;
            const float* bc = brow + cr;
            const float* cc = crow + cr;
            const float* mc = mrow + cr;
            const float* ac = arow + cr;
            const float* xc = xrow + cr;
            const float* zc = zrow + cg;
            float mx[MU], ax[AU];
            // PREP offsets: a per-lane base plus a multiple of the row stride that is the same for
            // every lane, so no per-lane multiply per load.
            const unsigned pb0 = static_cast<unsigned>((tid / N) * st32 + n_own);
            const unsigned px0 = static_cast<unsigned>(4 * g * st32 + col);
#pragma unroll
            for (int j = 0; j < BU; ++j) {
                const int t = (tid + NTH * j) / N;
                const unsigned off = PREP ? pb0 + static_cast<unsigned>(j * (NTH / N) * st32)
                                          : static_cast<unsigned>((t < Lc ? t : Lc - 1) * st32 + n_own);
                bx[j] = load_off32(bc, off);
                cx[j] = load_off32(cc, off);
            }
#pragma unroll
            for (int j = 0; j < MU; ++j) {
                if constexpr (PREP) break;
                const int u = tid + NTH * j;
                const int which = u < 3 * C ? u / C : 0, t = u % C;
                mx[j] = load_off32(mc, static_cast<unsigned>((t < Lc ? t : Lc - 1) * st32 + which * static_cast<int>(H)));
            }
            if (!PREP && R > 0) {
#pragma unroll
                for (int j = 0; j < AU; ++j) {
                    const unsigned u = static_cast<unsigned>(tid + NTH * j);
                    const unsigned uc = u < static_cast<unsigned>(C * R) ? u : static_cast<unsigned>(C * R - 1);
                    const int t = static_cast<int>((uc * rmagic) >> 16), r = static_cast<int>(uc) - t * R;
                    ax[j] = load_off32(ac, static_cast<unsigned>((t < Lc ? t : Lc - 1) * st32 + r));
                }
            }
#pragma unroll
            for (int st = 0; st < CT; ++st)
#pragma unroll
                for (int v = 0; v < 4; ++v) {
                    const int t = 16 * st + 4 * g + v;
                    const int tc = t < Lc ? t : Lc - 1;
                    if constexpr (PREP) {  // (the gate rows are the projection rows: gate = proj)
                        const unsigned off = px0 + static_cast<unsigned>((16 * st + v) * st32);
                        vx[st][v] = xc[off];
                        if (own(st, v)) zx[st][v] = zc[off];
                    } else {
                        vx[st][v] = load_off32(xc, static_cast<unsigned>(tc * st32 + col));
                        zx[st][v] = load_off32(zc, static_cast<unsigned>(tc * gst32 + col));
                    }
                }
#pragma unroll
            for (int j = 0; j < BU; ++j) {
                if constexpr (PREP) break;
                const int t = (tid + NTH * j) / N;
                k_sh[t * NP + n_own] = bx[j];
                q_sh[t * NP + n_own] = cx[j];
            }
#pragma unroll
            for (int j = 0; j < MU; ++j) {
                if constexpr (PREP) break;
                const int u = tid + NTH * j;
                if (u < 3 * C) raw_s[u / C][u % C] = mx[j];
            }
            if (!PREP && R > 0) {
#pragma unroll
                for (int j = 0; j < AU; ++j) {
                    const unsigned u = static_cast<unsigned>(tid + NTH * j);
                    const int t = static_cast<int>((u * rmagic) >> 16), r = static_cast<int>(u) - t * R;
                    if (u < static_cast<unsigned>(C * R)) ang_s[t * RM + r] = ax[j];
                }
            }
        }
        if constexpr (!PREP) __syncthreads();
        // b. Norm scales, coefficients, tanh(angle) * pi.
        if constexpr (PREP) {
            // Each wave forms the scales of the rows its threads scale in step c (rows 4 wave + q +
            // 8 j, q, j < 4), from the rows step a reads: lanes 0..15 the B rows, 16..31 the C rows.
            // Steps b and c then need no barrier.
            if (lane < 32) {
                const int k = lane & 15, t = 4 * wave + (k & 3) + 8 * (k >> 2);
                const bool isb = lane < 16;
                sc_s[isb ? 0 : 1][t] = bc_norm_scale_rows<N>((isb ? brow : crow) + t * static_cast<int>(a.st),
                                                             isb ? a.b_eps : a.c_eps);
            }
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
            __builtin_amdgcn_wave_barrier();
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        } else if (tid < 2 * C) {
            const int t = tid % C;
            const bool isb = tid < C;
            sc_s[isb ? 0 : 1][t] = bc_norm_scale_rows<N>((isb ? k_sh : q_sh) + t * NP, isb ? a.b_eps : a.c_eps);
        }
        // The coefficient wave (wave 1, or wave 0 when the block has one wave)
        // goes on to the decay weights (decay_walk). tanh runs on the other waves.
        if constexpr (!PREP) {
            const int ct = NTH >= 128 ? tid - 64 : tid;
            if (ct >= 0 && ct < C) token_coefficients<C>(ct, raw_s[0][ct], raw_s[1][ct], raw_s[2][ct], dt_bias, a.a_floor, Lc, coef);
            if (ct >= 0 && ct < 64) {
                // The coefficients above were written by other lanes of this wave.
                __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
                __builtin_amdgcn_wave_barrier();
                __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
            }
            decay_walk<C, (DT <= 2)>(ct, first, coef, w_s);
        }
        if constexpr (!PREP) {
            // tanh(angle) * pi on the waves other than the coefficient wave.
            const int tl = NTH >= 128 ? (tid < 64 ? tid : tid - 64) : tid;
            const bool tw = NTH < 128 || tid < 64 || tid >= 128;
            constexpr int TN = NTH >= 128 ? NTH - 64 : NTH;
            if (tw) {
#pragma unroll 1
                for (int i = tl; i < C * R; i += TN) {
                    const int t = static_cast<int>((static_cast<unsigned>(i) * rmagic) >> 16), r = i - t * R;
                    ang_s[t * RM + r] = tanhf_cr(ang_s[t * RM + r]) * kPiF;
                }
            }
        }
        if constexpr (PREP) {
            gates();
#pragma unroll
            for (int v = 0; v < kPrepOwnV; ++v) hooks.share_gate(v, gz[1][v]);
        } else if constexpr (kEarlyGate) {
            if (wave == 0) gates();  // wave 1 runs the coefficients and decay weights meanwhile
        }
        if constexpr (!PREP) __syncthreads();
        // c. q and k (all values read before any is written back); the
        //    running angle sums into cum_s; the decay weights.
        {
            constexpr int QU = C * N / NTH;
            float kv[QU], qv[QU], skb[QU], sqb[QU];
#pragma unroll
            for (int j = 0; j < QU; ++j) {
                const int t = (tid + NTH * j) / N, i = t * NP + n_own;
                kv[j] = PREP ? bx[j] : k_sh[i];
                qv[j] = PREP ? cx[j] : q_sh[i];
                skb[j] = sc_s[0][t];
                sqb[j] = sc_s[1][t];
            }
            const float bw = nrm_s[0][n_own], cw = nrm_s[1][n_own], bb = nrm_s[2][n_own], cb = nrm_s[3][n_own];
#pragma unroll
            for (int j = 0; j < QU; ++j) {
                const int t = (tid + NTH * j) / N, i = t * NP + n_own;
                k_sh[i] = (kv[j] * skb[j]) * bw + bb;
                q_sh[i] = (qv[j] * sqb[j]) * cw + cb;
            }
        }
        if (!PREP && tid < R) {
#pragma unroll
            for (int t0 = 0; t0 < C; t0 += 16) {
                float term[16];
#pragma unroll
                for (int i = 0; i < 16; ++i) term[i] = ang_s[(t0 + i) * RM + tid] * coef[3][t0 + i];
#pragma unroll
                for (int i = 0; i < 16; ++i) {
                    running += static_cast<double>(term[i]);
                    cum_s[(t0 + i) * RM + tid] = static_cast<float>(running);
                }
            }
        }
        if constexpr (kEarlyGate && !PREP) {
            if (wave == 1) gates();  // wave 0 runs the angle sums meanwhile
        }
        // d. Rotation of the (2r, 2r + 1) pairs. PREP: each wave rotates the rows it scaled in step
        //    c, once the rotations are in (hooks.wait_rotations), with no barrier before.
        auto rotate = [&](int t, int r, float sine, float cosine) {
            float* qp = q_sh + t * NP + 2 * r;
            float* kq = k_sh + t * NP + 2 * r;
            const float ql = qp[0], qr = qp[1], kl = kq[0], kr = kq[1];
            qp[0] = fmaf(ql, cosine, -(qr * sine));
            qp[1] = fmaf(ql, sine, qr * cosine);
            kq[0] = fmaf(kl, cosine, -(kr * sine));
            kq[1] = fmaf(kl, sine, kr * cosine);
        };
        if constexpr (PREP) {
            // The pairs were scaled in step c by other lanes of this wave.
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
            __builtin_amdgcn_wave_barrier();
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
            hooks.wait_rotations();
            const float* rot = hooks.rotations();
#pragma unroll 1
            for (int i = lane; i < 16 * R; i += 64) {
                const int k = static_cast<int>((static_cast<unsigned>(i) * rmagic) >> 16), r = i - k * R;
                const int t = 4 * wave + (k & 3) + 8 * (k >> 2);
                rotate(t, r, rot[2 * (t * RM + r)], rot[2 * (t * RM + r) + 1]);
            }
        } else {
            __syncthreads();
#pragma unroll 1
            for (int i = tid; i < C * R; i += NTH) {
                const int t = static_cast<int>((static_cast<unsigned>(i) * rmagic) >> 16), r = i - t * R;
                float sine, cosine;
                rotation_of(cum_s[t * RM + r], &sine, &cosine);
                rotate(t, r, sine, cosine);
            }
        }
        __syncthreads();
        static_assert(!PREP || CT == 2, "PREP: two token tiles");
        // e. Masked G^T tiles into LDS (tile pair p on wave p % DT); ck; k_p. PREP (one chunk, the
        //    first and last): every wave forms token tile 0's pair into registers (pg), the products
        //    and rounding of the LDS form, and goes straight on to its outputs.
        f32x4_t pg[PREP ? NPAIR : 1];
        {
            int p = 0;
#pragma unroll
            for (int tt = 0; tt < CTE; ++tt) {
#pragma unroll
                for (int st = 0; st <= tt; ++st, ++p) {
                    // (PREP forms every tile: rows past the end hold the last token's values, and
                    // the tiles stay one straight block whose product chains interleave.)
                    if (!PREP && (p % DT != wave || 16 * tt >= Lc)) continue;
                    f32x4_t acc = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
                    for (int nt = 0; nt < NT; ++nt) {
                        const float4 k4 = *reinterpret_cast<const float4*>(k_sh + (16 * st + li) * NP + 16 * nt + 4 * g);
                        const float4 q4 = *reinterpret_cast<const float4*>(q_sh + (16 * tt + li) * NP + 16 * nt + 4 * g);
                        acc = __builtin_amdgcn_mfma_f32_16x16x4f32(k4.x, q4.x, acc, 0, 0, 0);
                        acc = __builtin_amdgcn_mfma_f32_16x16x4f32(k4.y, q4.y, acc, 0, 0, 0);
                        acc = __builtin_amdgcn_mfma_f32_16x16x4f32(k4.z, q4.z, acc, 0, 0, 0);
                        acc = __builtin_amdgcn_mfma_f32_16x16x4f32(k4.w, q4.w, acc, 0, 0, 0);
                    }
                    const float4 w4 = *reinterpret_cast<const float4*>(w_s + (16 * tt + li) * WP + 16 * st + 4 * g);
                    f32x4_t pv = f32x4_t{w4.x * acc[0], w4.y * acc[1], w4.z * acc[2], w4.w * acc[3]};
                    if (st == tt) {  // W[t][s] is defined for s <= t only
#pragma unroll
                        for (int v = 0; v < 4; ++v) pv[v] = 4 * g + v <= li ? pv[v] : 0.0f;
                    }
                    if constexpr (PREP)
                        pg[p] = pv;
                    else
                        p_s[p * 64 + lane] = pv;
                }
            }
        }
        if constexpr (!PREP) {
            if (!first && wave == DT - 1 && lane < C) {  // (read for later chunks only)
                float dot = 0.0f;
#pragma unroll
                for (int n = 0; n < N; ++n) dot = fmaf(q_sh[lane * NP + n], kp_s[par][n], dot);
                ck_s[lane] = dot * w_s[lane * WP + kWp];
            }
            if (tid < N) kp_s[par ^ 1][tid] = k_sh[(C - 1) * NP + tid];
            __syncthreads();
        }
        // f. This wave's output columns (gates formed above for two-wave
        //    blocks, here otherwise). PREP (the first chunk: no carried
        //    state): token tile 0's products first, then its outputs, so
        //    the predicated stores do not split the product chains.
        if constexpr (PREP) {
            f32x4_t Y[CTE];
            int p0 = 0;
#pragma unroll
            for (int tt = 0; tt < CTE; ++tt) {
                Y[tt] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int st = 0; st <= tt; ++st)
#pragma unroll
                    for (int v = 0; v < 4; ++v)
                        Y[tt] = __builtin_amdgcn_mfma_f32_16x16x4f32(pg[p0 + st][v], vx[st][v], Y[tt], 0, 0, 0);
                p0 += tt + 1;
            }
            float o[CTE][4];
#pragma unroll
            for (int tt = 0; tt < CTE; ++tt)
#pragma unroll
                for (int v = 0; v < 4; ++v) {
                    const float y = fmaf(skip, vx[tt][v], Y[tt][v]);
                    o[tt][v] = static_cast<float>(static_cast<double>(y) * gz[tt][v]);
                }
            // 32-bit row offsets from this lane's column (C rows of d_inner floats); a whole chunk
            // stores without per-lane predication.
            float* ocol = orow + col;
            const int di = static_cast<int>(d_inner);
            if (Lc == C) {
#pragma unroll
                for (int tt = 0; tt < CTE; ++tt)
#pragma unroll
                    for (int v = 0; v < 4; ++v) store_off32(ocol, static_cast<unsigned>((16 * tt + 4 * g + v) * di), o[tt][v]);
            } else {
#pragma unroll
                for (int tt = 0; tt < CTE; ++tt)
#pragma unroll
                    for (int v = 0; v < 4; ++v) {
                        const int t = 16 * tt + 4 * g + v;
                        if (t < Lc) store_off32(ocol, static_cast<unsigned>(t * di), o[tt][v]);
                    }
            }
        } else {
            if constexpr (!kEarlyGate) gates();
            // 32-bit offsets from the chunk's first output row (C rows of d_inner floats).
            float* ochunk = orow + (TILE_OUT ? 0 : c0) * d_inner;
            const int di = static_cast<int>(d_inner);
            int p0 = 0;  // index of pair (tt, 0)
#pragma unroll
            for (int tt = 0; tt < CT; ++tt) {
                const int t0 = 16 * tt;
                if (t0 < Lc) {
                    f32x4_t Y = f32x4_t{0.f, 0.f, 0.f, 0.f}, Yi = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
                    for (int st = 0; st <= tt; ++st) {
                        const f32x4_t P = p_s[(p0 + st) * 64 + lane];
#pragma unroll
                        for (int v = 0; v < 4; ++v) Y = __builtin_amdgcn_mfma_f32_16x16x4f32(P[v], vx[st][v], Y, 0, 0, 0);
                    }
#pragma unroll
                    for (int nt = 0; nt < NT; ++nt) {
                        const float4 q4 = *reinterpret_cast<const float4*>(q_sh + (t0 + li) * NP + 16 * nt + 4 * g);
                        const float qv[4] = {q4.x, q4.y, q4.z, q4.w};
#pragma unroll
                        for (int v = 0; v < 4; ++v) Yi = __builtin_amdgcn_mfma_f32_16x16x4f32(qv[v], S[nt][v], Yi, 0, 0, 0);
                    }
#pragma unroll
                    for (int v = 0; v < 4; ++v) {
                        const int t = t0 + 4 * g + v;
                        const float yc = fmaf(ck_s[t], vp, fmaf(w_s[t * WP + kDin], Yi[v], Y[v]));
                        float y = first ? Y[v] : yc;
                        y = fmaf(skip, vx[tt][v], y);
                        // With an explicit gate gz = z, and the double product of two
                        // floats rounded once is the fp32 product y * gate.
                        const float o = static_cast<float>(static_cast<double>(y) * gz[tt][v]);
                        if (!last || t < Lc) store_off32(ochunk, static_cast<unsigned>(t * di + col), o);
                    }
                }
                p0 += tt + 1;
            }
        }
        if constexpr (last) return;
        // g. This wave's state columns after the chunk (all C tokens valid).
        {
            const float dl = w_s[(C - 1) * WP + kDin], wl = w_s[(C - 1) * WP + kWp];
#pragma unroll
            for (int nt = 0; nt < NT; ++nt)
#pragma unroll
                for (int v = 0; v < 4; ++v) {
                    float x = S[nt][v] * dl;
                    x = fmaf(wl * kp_s[par][16 * nt + 4 * g + v], vp, x);  // k_p, v_p are zero in the first chunk
                    S[nt][v] = x;
                }
#pragma unroll
            for (int st = 0; st < CT; ++st) {
                float kA[4][NT], bv[4];
#pragma unroll
                for (int v = 0; v < 4; ++v) {
                    const int srow = 16 * st + 4 * g + v;
                    bv[v] = w_s[(C - 1) * WP + srow] * vx[st][v];
#pragma unroll
                    for (int nt = 0; nt < NT; ++nt) kA[v][nt] = k_sh[srow * NP + 16 * nt + li];
                }
#pragma unroll
                for (int v = 0; v < 4; ++v)
#pragma unroll
                    for (int nt = 0; nt < NT; ++nt) S[nt] = __builtin_amdgcn_mfma_f32_16x16x4f32(kA[v][nt], bv[v], S[nt], 0, 0, 0);
            }
            vp = __shfl(vx[CT - 1][3], 48 + li, 64);
        }
        __syncthreads();
    };
    int64_t c0 = 0;
    for (; c0 + C < L; c0 += C) {
        hooks.before(c0);
        chunk(std::false_type{}, c0);
        hooks.after(c0, false);
    }
    hooks.before(c0);
    chunk(std::true_type{}, c0);
    hooks.after(c0, true);
}

// One block of DT waves per (window, head). Four waves per SIMD for the
// four-wave blocks: at d_state 64 the compiler then spills 8 VGPRs, and the
// kernel is 5% faster than at three waves (1.17 vs 1.23 ms at 1024 x 256
// tokens, 8 heads); the others as they fall. Blocks are ordered so that the
// heads of one window run on one XCD and share its L2 copy of the window's
// B/C rows.
template <int C, int NT, int DT>
__global__ __launch_bounds__(64 * DT) __attribute__((amdgpu_waves_per_eu(DT == 4 ? 4 : 1)))
void scan_fused_kernel(ScanArgs a) {
    __shared__ ScanLds<C, NT, DT> sh;
    // Block -> (window, head) in 32-bit arithmetic (B * H < 2^31, checked at launch).
    const unsigned Hu = static_cast<unsigned>(a.H), nblk = static_cast<unsigned>(a.B * a.H);
    unsigned lin = blockIdx.x;
    if (nblk % 8 == 0) lin = (lin % 8) * (nblk / 8) + lin / 8;
    scan_head<C, NT, DT, false>(a, sh, lin / Hu, lin % Hu, 0, NoChunkHooks{});
}

bool aligned16(const void* ptr) { return (reinterpret_cast<uintptr_t>(ptr) & 15) == 0; }

// MLK_MAMBA3_SCAN selects the forward's scan: unset (or "fused") the fused
// kernel where the geometry allows it; "unfused" prep -> rotate -> recurrence
// kernel (chunked or time-sequential by the rule in launch_rec); "sequential"
// prep -> rotate -> the time-sequential kernel, the reference's association.
enum class ScanMode { kFused, kUnfused, kSequential };

ScanMode scan_mode() {
    const char* mode = std::getenv("MLK_MAMBA3_SCAN");
    if (mode == nullptr) return ScanMode::kFused;
    if (std::strcmp(mode, "sequential") == 0) return ScanMode::kSequential;
    if (std::strcmp(mode, "unfused") == 0) return ScanMode::kUnfused;
    return ScanMode::kFused;
}

bool launch_scan_fused(const ScanArgs& s, int64_t N, int64_t D, hipStream_t stream) {
    const int NT = static_cast<int>(N / 16), DT = static_cast<int>(D / 16);
    const dim3 grid(static_cast<unsigned>(s.B * s.H));
#define MLK_FUSED(NTV, DTV)                                                                                  \
    if (NT == NTV && DT == DTV) {                                                                            \
        hipLaunchKernelGGL((scan_fused_kernel<32, NTV, DTV>), grid, dim3(64 * DTV), 0, stream, s);          \
        return true;                                                                                         \
    }
    MLK_FUSED(1, 1) MLK_FUSED(1, 2) MLK_FUSED(1, 4) MLK_FUSED(2, 1) MLK_FUSED(2, 2) MLK_FUSED(2, 4)
    MLK_FUSED(4, 1) MLK_FUSED(4, 2) MLK_FUSED(4, 4)
#undef MLK_FUSED
    return false;
}

// ---------------------------------------------------------------------------
// The RMSNorm -> Mamba-3 block: GroupedRMSNorm + in_proj + scan in one kernel
// ---------------------------------------------------------------------------
//
// x + out_proj(mixer(in_proj(GroupedRMSNorm(x)))) (the Mamba3Layer forward of
// reference/Model/layers/mamba3_layer.py:488-498 over mamba3_siso_layer,
// montlok.cpp:496-519) in two launches: this kernel (the block's mixer,
// mlk_rms_norm_mamba3_forward), then the out_proj with the residual added in
// its epilogue (mlk_linear_residual). One block
// of DT waves per (window, head), so that each head's scan keeps a SIMD to
// itself, as in scan_fused_kernel. Per 32-token chunk, before the scan, the
// block computes the in_proj columns its head reads (its z and x columns, the
// B/C group rows, the dt/A/trap logits and the angles: 7 column tiles at the
// block workload's geometry, against 19 for the whole row) for the chunk's
// rows into LDS, laid out as the whole row; each wave normalises its x
// fragments of the chunk's two 16-row tiles once and computes 16 x 16 tiles
// with the arithmetic of the one-wave-per-tile linear and its GroupedRMSNorm
// prologue (tile_f32.h). scan_head then reads the rows from LDS and writes the
// gated outputs y [B, L, d_inner]. The in_proj rows never reach HBM; the
// result equals rms_norm_linear -> mamba3_siso_forward bit for bit wherever
// the former takes its one-wave-per-tile form.
struct BlockArgs {
    const float* x;  // [B, L, dm], token rows x_ts floats apart, windows x_bs apart
    int64_t x_bs, x_ts;
    int64_t dm, W;
    const float* norm_w;  // [dm]
    double norm_eps;
    const float* in_w;  // [W, dm] fp32
    ScanArgs s;         // mixer parameters, B, L, G, H, R and the output y (proj and gate are set in the kernel)
};

// HELP (one chunk, L <= 32; the dt/A/trap/angle columns one column tile, the
// last): the block has DT more waves. The DT scan waves compute the other
// column tiles of their row tile (wave w: rows 16 w .. 16 w + 15) but the
// last two; each helper computes the last tile for all 32 rows (helper 1 the
// second-to-last beside it) and, from it, helper 0 the chunk's step
// coefficients and then its decay weights, helper 1 tanh(angle) * pi, then
// the running angle sums and rotations, and helper 0 some of the gates, while the
// scan waves copy their rows, form the norm scales and the other gates
// (scan_head's PREP form). After the barrier that ends step d each helper
// forms token tile 1's outputs of one head column tile while the scan waves
// form tile 0's, and ends.
// i / R as (i * hmagic(R)) >> 16, exact for i < 2^10 and 0 < R <= 32 (the helpers' (token, angle) item
// indices, i < C * R <= 256): a multiply and a shift instead of the integer division's VALU sequence.
__device__ __forceinline__ unsigned hmagic(int R) { return (65536u + static_cast<unsigned>(R) - 1u) / static_cast<unsigned>(R); }

template <int NT, int DT, int KSI, int GS, int NCT, bool ALL_LIVE, bool HELP>
__global__ __launch_bounds__(64 * DT * (HELP ? 2 : 1)) __attribute__((amdgpu_waves_per_eu(1)))
void mamba3_block_scan_kernel(BlockArgs p) {
    constexpr int C = 32, D = 16 * DT;
    constexpr bool STAGE = ALL_LIVE && KSI == 2;  // d_model 64: the weight rows staged in LDS
    __shared__ __attribute__((aligned(16))) float w_lds[STAGE ? NCT * 16 * 64 : 4];
    static_assert(DT == 2, "one wave per 16-row tile of the 32-token chunk");
    __shared__ ScanLds<C, NT, DT> sh;
    constexpr int HP = 17;  // helper staging: [32 rows][16 columns], rows HP floats apart
    __shared__ __attribute__((aligned(16))) float hs[HELP ? DT : 1][HELP ? C * HP : 1];
    __shared__ int rot_ready;  // HELP: set by helper 1 once the rotations are in hs[1]
    __shared__ double lg[HELP ? DT * 4 * 64 : 1];  // HELP: token tile 1's gates, [scan wave][v][lane]
    extern __shared__ __attribute__((aligned(16))) float proj_s[];  // [C, pp]

    const int64_t H = p.s.H, L = p.s.L;
    // Block -> (window, head), the heads of a window on one XCD (as scan_fused_kernel).
    const unsigned Hu = static_cast<unsigned>(H), nblk = static_cast<unsigned>(p.s.B * H);
    unsigned lin = blockIdx.x;
    if (nblk % 8 == 0) lin = (lin % 8) * (nblk / 8) + lin / 8;
    const int64_t b = lin / Hu, h = lin % Hu;
    const int lane = threadIdx.x & 63, li = lane & 15, grp = lane >> 4;
    const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x) >> 6);
    const int dm = static_cast<int>(p.dm), W = static_cast<int>(p.W);
    const int DI = static_cast<int>(H) * D;
    const int pp = (W + 15) / 16 * 16 + 4;
    const float* xw = p.x + b * p.x_bs;

    ScanArgs a = p.s;
    a.proj = proj_s;
    a.sb = 0;
    a.st = pp;
    a.gate = proj_s;
    a.gsb = 0;
    a.gst = pp;
    a.gate_logits = 1;

    struct Hooks {
        const BlockArgs& p;
        const float* xw;
        float* proj_s;
        float* w_lds;
        int64_t L;
        int li, grp, wave, dm, W, DI, pp, h;

        // This head's column tiles: z (D / 16), x (D / 16), the B/C rows, then
        // dt/A/trap/angles to the end of the row.
        __device__ int tile_col(int j) const {
            constexpr int DTL = D / 16;
            if (j < DTL) return h * D + 16 * j;
            if (j < 2 * DTL) return DI + h * D + 16 * (j - DTL);
            return 2 * DI + 16 * (j - 2 * DTL);
        }

        // STAGE (d_model 64): before the first chunk the block copies the
        // head's weight rows into LDS with direct global-to-LDS loads (each
        // instruction moves four 256-byte rows; no registers, all in flight
        // at once, each row read from L2 once per block instead of once per
        // wave); row r of tile j holds its 16-byte chunk c at slot c ^ r, so
        // the 16 lanes of a fragment read hit 16 different bank groups.
        // stage_issue puts the copies in flight (a compile-time count per wave, so the waits the
        // compiler places for the x fragments leave them outstanding: the norm of x runs while they
        // land); stage_wait waits for them and for the other waves'.
        __device__ void stage_issue(int ncol) const {
            if constexpr (STAGE) {
                static_assert(KSI == 2 && ALL_LIVE, "staging takes d_model 64 rows: 16 chunks of 16 bytes");
                constexpr int NW = HELP ? 2 * DT : DT;
                static_assert((4 * NCT) % NW == 0, "every wave issues the same number of quarter tiles");
                const int lane = threadIdx.x & 63;
                const int rq = lane >> 4, slot = lane & 15;
#pragma unroll
                for (int k = 0; k < 4 * NCT / NW; ++k) {  // quarter-tile u: tile u / 4, rows 4 (u % 4) ..
                    const int u = wave + k * NW;
                    const int j = u >> 2, row = 4 * (u & 3) + rq;
                    const int n = tile_col(j < ncol ? j : ncol - 1) + row;
                    const unsigned off = static_cast<unsigned>((n < W ? n : W - 1) * 64 + 4 * (slot ^ row)) << 2;
                    const float* src = reinterpret_cast<const float*>(reinterpret_cast<const char*>(p.in_w) + off);
                    __builtin_amdgcn_global_load_lds(
                        (const __attribute__((address_space(1))) void*)src,
                        (__attribute__((address_space(3))) void*)(w_lds + u * 256), 16, 0, 0);
                }
            }
        }
        // The normalised fragments are pinned before the barrier: left to itself the compiler
        // schedules part of the norm after it, where it delays the first products.
        __device__ static void hold(float (&v)[KSI][8]) {
#pragma unroll
            for (int s2 = 0; s2 < KSI; ++s2)
#pragma unroll
                for (int k = 0; k < 8; ++k) asm volatile("" : "+v"(v[s2][k]));
        }
        __device__ void stage_wait() const {
            if constexpr (STAGE) {
                __builtin_amdgcn_s_waitcnt(0);  // vmcnt(0) expcnt(0) lgkmcnt(0): the LDS copies have landed
                __syncthreads();
            }
        }

        // Column tile j's 16 weight rows as this lane's fragments (lane l = 16 g + i: row i, k = 32 s + 8 g ..).
        __device__ void weights(int j, int ncol, float (&wv)[KSI][8], bool (&wlive)[KSI]) const {
            if constexpr (STAGE) {
                const float* rowp = w_lds + ((j < NCT ? j : NCT - 1) * 16 + li) * 64;
#pragma unroll
                for (int s2 = 0; s2 < KSI; ++s2) {
                    const int cc = 8 * s2 + 2 * grp;
                    const float4 lo = *reinterpret_cast<const float4*>(rowp + 4 * (cc ^ li));
                    const float4 hi = *reinterpret_cast<const float4*>(rowp + 4 * ((cc + 1) ^ li));
                    wv[s2][0] = lo.x; wv[s2][1] = lo.y; wv[s2][2] = lo.z; wv[s2][3] = lo.w;
                    wv[s2][4] = hi.x; wv[s2][5] = hi.y; wv[s2][6] = hi.z; wv[s2][7] = hi.w;
                    wlive[s2] = true;
                }
            } else {
                const int n0 = tile_col(j < ncol ? j : ncol - 1);
                const int wr = n0 + li < W ? n0 + li : W - 1;
                tile_load8<KSI>(p.in_w + static_cast<int64_t>(wr) * dm, dm, grp, wv, wlive);
            }
        }

        // The chunk's in_proj tiles into proj_s, then a barrier. Without
        // HELP, wave w computes the chunk's 16-row tile w % 2 against the
        // head's column tiles j = w / 2, w / 2 + NW / 2, ... (NW = DT); with
        // HELP (scan waves only), row tile w against every tile but the last two.
        // The tiles past the head's count repeat its last one and are not
        // stored. Every wave normalises its x fragments once; all of its
        // weight loads are in flight before the first wait.
        __device__ void before(int64_t c0) const {
            constexpr int NTW = HELP ? NCT - 2 : (NCT + DT / 2 - 1) / (DT / 2);  // column tiles per wave
            const int ncol = 2 * (D / 16) + (W - 2 * DI + 15) / 16;
            const int rt = HELP ? wave : wave & 1, j0 = HELP ? 0 : wave >> 1, jstep = HELP ? 1 : DT / 2;
            float xv[KSI][8], nw[KSI][8];
            bool live[KSI], nlive[KSI];
            const int64_t r = c0 + 16 * rt + li;
            tile_load8<KSI>(xw + (r < L ? r : L - 1) * p.x_ts, dm, grp, xv, live);
            tile_load8<KSI>(p.norm_w, dm, grp, nw, nlive);
            // (HELP runs one chunk, c0 = 0: no branch, so the compiler's wait for x leaves the
            // copies outstanding.)
            if (HELP || c0 == 0) stage_issue(ncol);
            if constexpr (STAGE) {
                tile_rms_norm<KSI, GS>(xv, nw, p.norm_eps);  // while the weight rows land
                hold(xv);
                if (HELP || c0 == 0) stage_wait();
            }
            float wv[NTW][KSI][8];
            bool wlive[NTW][KSI];
#pragma unroll
            for (int i = 0; i < NTW; ++i) weights(j0 + i * jstep, ncol, wv[i], wlive[i]);
            if constexpr (!STAGE) {
                // Every loaded value is held here, so all the loads are in
                // flight together and waited on once: left to itself the
                // compiler issues the later tiles' loads after the first
                // products (or after the norm) and waits on each batch in turn.
#pragma unroll
                for (int s2 = 0; s2 < KSI; ++s2)
#pragma unroll
                    for (int k = 0; k < 8; ++k)
#pragma unroll
                        for (int i = 0; i < NTW; ++i) asm volatile("" : "+v"(wv[i][s2][k]));
                tile_rms_norm<KSI, GS>(xv, nw, p.norm_eps);
            }
            auto put = [&](int i, tile_f32x4 y) {
                const int j = j0 + i * jstep;
                y += tile_f32x4{0.0f, 0.0f, 0.0f, 0.0f};  // the linear's (zero) bias add
                // (HELP: every tile of the scan waves lies below ncol = NCT, checked at launch, so the
                // store needs no branch and stays in one block with the products.)
                if (HELP || j < ncol) *reinterpret_cast<tile_f32x4*>(proj_s + (16 * rt + li) * pp + tile_col(j) + 4 * grp) = y;
            };
            // Two tiles' chains interleaved per pair; a pair's results are summed and stored after the
            // next pair's products are issued, so the accumulator reads do not drain the matrix core.
            tile_f32x4 pa, pb;
#pragma unroll
            for (int i = 0; i + 1 < NTW; i += 2) {
                tile_f32x4 ya, yb;
                tile_mfma_f32_pair<KSI, ALL_LIVE>(wv[i], wv[i + 1], xv, live, ya, yb);
                if (i > 0) {
                    put(i - 2, pa);
                    put(i - 1, pb);
                }
                pa = ya;
                pb = yb;
            }
            if constexpr (NTW % 2 == 1) {
                const tile_f32x4 y = tile_mfma_f32<KSI, ALL_LIVE>(wv[NTW - 1], xv, live);
                if constexpr (NTW > 1) {
                    put(NTW - 3, pa);
                    put(NTW - 2, pb);
                }
                put(NTW - 1, y);
            } else {
                put(NTW - 2, pa);
                put(NTW - 1, pb);
            }
            __syncthreads();
        }
        __device__ void after(int64_t, bool) const {}
        __device__ const float* rotations() const { return rot; }
        // The scan waves' wait for helper 1's rotations: it sets the flag after writing them, with
        // nothing in between that waits on the scan waves, so the wait ends.
        __device__ void wait_rotations() const {
            while (__hip_atomic_load(ready, __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_WORKGROUP) == 0)
                __builtin_amdgcn_s_sleep(1);
        }
        // A scan wave's tile-1 gate v (< kPrepOwnV) of this lane, for the helper that forms the outputs.
        __device__ void share_gate(int v, double gate) const { gates[(wave * 4 + v) * 64 + (threadIdx.x & 63)] = gate; }
        const float* rot;
        int* ready;
        double* gates;
    };
    if (threadIdx.x == 0) rot_ready = 0;  // read after the in_proj barrier, set after it
    const Hooks hooks{p,  xw, proj_s, w_lds, L,  li, grp, wave, dm, W, DI, pp, static_cast<int>(h), &hs[HELP ? 1 : 0][0],
                      &rot_ready, lg};
    if constexpr (HELP) {
        if (wave >= DT) {
            // The last column tile (dt, A, trap logits, angles) for both row tiles into this helper's
            // staging rows, with the scan waves' arithmetic.
            const int ncol = 2 * (D / 16) + (W - 2 * DI + 15) / 16;
            const int j = ncol - 1, hw = wave - DT;
            float nw[KSI][8], wv[KSI][8];
            bool nlive[KSI], wlive[KSI];
            float xv[2][KSI][8];
            bool live[2][KSI];
#pragma unroll
            for (int rt = 0; rt < 2; ++rt) {
                const int64_t r = 16 * rt + li;
                tile_load8<KSI>(xw + (r < L ? r : L - 1) * p.x_ts, dm, grp, xv[rt], live[rt]);
            }
            tile_load8<KSI>(p.norm_w, dm, grp, nw, nlive);
            hooks.stage_issue(ncol);
#pragma unroll
            for (int rt = 0; rt < 2; ++rt) {
                tile_rms_norm<KSI, GS>(xv[rt], nw, p.norm_eps);
                hooks.hold(xv[rt]);
            }
            hooks.stage_wait();
            hooks.weights(j, ncol, wv, wlive);
            // Helper 1 also computes the second-to-last tile (the C rows) for both row tiles, its
            // chains interleaved with the last tile's; the scan waves skip it.
            float wc[KSI][8];
            bool wclive[KSI];
            if (hw == 1) hooks.weights(j - 1, ncol, wc, wclive);
            // Both row tiles' products first, then the stores (in one block, the row tiles' chains
            // interleave and the accumulator reads do not drain the matrix core between them).
            tile_f32x4 y[2];
            if (hw == 1) {
                tile_f32x4 yc[2];
#pragma unroll
                for (int rt = 0; rt < 2; ++rt) tile_mfma_f32_pair<KSI, ALL_LIVE>(wv, wc, xv[rt], live[rt], y[rt], yc[rt]);
#pragma unroll
                for (int rt = 0; rt < 2; ++rt) {
                    yc[rt] += tile_f32x4{0.0f, 0.0f, 0.0f, 0.0f};  // the linear's (zero) bias add
                    *reinterpret_cast<tile_f32x4*>(proj_s + (16 * rt + li) * pp + hooks.tile_col(j - 1) + 4 * grp) = yc[rt];
                }
            } else {
#pragma unroll
                for (int rt = 0; rt < 2; ++rt) y[rt] = tile_mfma_f32<KSI, ALL_LIVE>(wv, xv[rt], live[rt]);
            }
#pragma unroll
            for (int rt = 0; rt < 2; ++rt) {
                y[rt] += tile_f32x4{0.0f, 0.0f, 0.0f, 0.0f};  // the linear's (zero) bias add
#pragma unroll
                for (int v = 0; v < 4; ++v) hs[hw][(16 * rt + li) * HP + 4 * grp + v] = y[rt][v];
            }
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
            __builtin_amdgcn_wave_barrier();
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
            // Column offsets inside the tile: dt h, A H + h, trap 2H + h, angle r 3H + r. Tokens past L
            // hold the last token's values (their x rows are clamped), as the scan's own copy reads them.
            const int Hi = static_cast<int>(H), Lc = static_cast<int>(L);
            const float* row = hs[hw];
            if (hw == 0) {
                if (lane < C)
                    token_coefficients<C>(lane, row[lane * HP + h], row[lane * HP + Hi + h], row[lane * HP + 2 * Hi + h],
                                          p.s.dt_bias[h], p.s.a_floor, Lc, sh.coef);
            } else if (lane < C * static_cast<int>(p.s.R)) {
                // tanh(angle) * pi of the first 64 (token, angle) items; the rest after the barrier, where
                // this helper has slack and the scan waves do not wait for it.
                const int R = static_cast<int>(p.s.R);
                constexpr int RM = ScanLds<C, NT, DT>::RM;
                const int t = static_cast<int>((static_cast<unsigned>(lane) * hmagic(R)) >> 16), rr = lane - t * R;
                sh.ang_s[t * RM + rr] = tanhf_cr(row[t * HP + 3 * Hi + rr]) * kPiF;
            }
            __syncthreads();  // with the end of the scan waves' in_proj: the coefficients are in
            if (hw == 0) {
                decay_walk<C, true>(lane, true, sh.coef, sh.w_s);
            } else {
                // The remaining tanh(angle) * pi items, then the running angle sums of the chunk (one lane
                // per angle, from zero: the first chunk) as step c forms them: each term tanh(angle) * pi
                // * dt in fp32, widened, added in token order in fp64, the sum rounded to fp32 where it is
                // used. The terms are formed for every item at once, in helper 0's staging rows (dead after
                // the barrier), so the lanes that walk the sums only add and store; then the sin/cos of
                // every (token, angle) pair, as step d would, into this helper's staging rows (its tile
                // values are dead by then).
                const int R = static_cast<int>(p.s.R);
                constexpr int RM = ScanLds<C, NT, DT>::RM;
                static_assert(sizeof(double) * C * RM <= sizeof(float) * C * HP, "the sums fit the staging rows");
                double* cum_d = reinterpret_cast<double*>(&hs[0][0]);
                if (lane < C * R) {  // items 0 .. 63: tanh formed before the barrier
                    const int t = static_cast<int>((static_cast<unsigned>(lane) * hmagic(R)) >> 16), rr = lane - t * R;
                    cum_d[t * RM + rr] = static_cast<double>(sh.ang_s[t * RM + rr] * sh.coef[3][t]);
                }
#pragma unroll 1
                for (int i = lane + 64; i < C * R; i += 64) {
                    const int t = static_cast<int>((static_cast<unsigned>(i) * hmagic(R)) >> 16), rr = i - t * R;
                    const float a = tanhf_cr(row[t * HP + 3 * Hi + rr]) * kPiF;
                    cum_d[t * RM + rr] = static_cast<double>(a * sh.coef[3][t]);
                }
                __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
                __builtin_amdgcn_wave_barrier();
                __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
                if (lane < R) {
                    double term[C];
#pragma unroll
                    for (int t = 0; t < C; ++t) term[t] = cum_d[t * RM + lane];
                    double running = 0.0;
#pragma unroll
                    for (int t = 0; t < C; ++t) {
                        running += term[t];
                        cum_d[t * RM + lane] = running;
                    }
                }
                __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
                __builtin_amdgcn_wave_barrier();
                __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
                float* rot = hs[1];
                static_assert(2 * C * RM <= C * HP, "the rotations fit the staging rows");
#pragma unroll 1
                for (int i = lane; i < C * R; i += 64) {
                    const int t = static_cast<int>((static_cast<unsigned>(i) * hmagic(R)) >> 16), rr = i - t * R;
                    rotation_of(static_cast<float>(cum_d[t * RM + rr]), &rot[2 * (t * RM + rr)], &rot[2 * (t * RM + rr) + 1]);
                }
                __hip_atomic_store(&rot_ready, 1, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_WORKGROUP);
            }
            // Helper 0 (done with its decay weights well before helper 1's rotations) forms the other
            // token tile 1 gates of both column tiles (v >= kPrepOwnV: tokens 16 + 4 grp + v, head column
            // 16 sw + li), as scan_head forms them from z (the head's first columns of the rows; the
            // tile's rows past the end hold the last token's).
            if (hw == 0) {
#pragma unroll
                for (int sw = 0; sw < DT; ++sw)
#pragma unroll
                    for (int v = kPrepOwnV; v < 4; ++v) {
                        const double z = static_cast<double>(
                            proj_s[(16 + 4 * grp + v) * pp + static_cast<int>(h) * D + 16 * sw + li]);
                        lg[(sw * 4 + v) * 64 + lane] = silu_d(z);
                    }
            }
            __syncthreads();  // with the end of the scan waves' step d: decay weights, gates, q and k are in
            // Token tile 1's outputs of head column tile hw (tokens 16 + 4 grp + v, column 16 hw + li), as
            // scan_head's steps e and f form them: the masked G^T tiles (1, 0) and (1, 1) from the scaled and
            // rotated q/k rows and the decay weights, their products with x in the same order, the skip term
            // and the gate (the scan waves take tile 0).
            {
                using SL = ScanLds<C, NT, DT>;
                f32x4_t pg[2];
#pragma unroll
                for (int st = 0; st < 2; ++st) {
                    f32x4_t acc = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
                    for (int nt = 0; nt < NT; ++nt) {
                        const float4 k4 = *reinterpret_cast<const float4*>(sh.k_sh + (16 * st + li) * SL::NP + 16 * nt + 4 * grp);
                        const float4 q4 = *reinterpret_cast<const float4*>(sh.q_sh + (16 + li) * SL::NP + 16 * nt + 4 * grp);
                        acc = __builtin_amdgcn_mfma_f32_16x16x4f32(k4.x, q4.x, acc, 0, 0, 0);
                        acc = __builtin_amdgcn_mfma_f32_16x16x4f32(k4.y, q4.y, acc, 0, 0, 0);
                        acc = __builtin_amdgcn_mfma_f32_16x16x4f32(k4.z, q4.z, acc, 0, 0, 0);
                        acc = __builtin_amdgcn_mfma_f32_16x16x4f32(k4.w, q4.w, acc, 0, 0, 0);
                    }
                    const float4 w4 = *reinterpret_cast<const float4*>(sh.w_s + (16 + li) * SL::WP + 16 * st + 4 * grp);
                    f32x4_t pv = f32x4_t{w4.x * acc[0], w4.y * acc[1], w4.z * acc[2], w4.w * acc[3]};
                    if (st == 1) {  // W[t][s] is defined for s <= t only
#pragma unroll
                        for (int v = 0; v < 4; ++v) pv[v] = 4 * grp + v <= li ? pv[v] : 0.0f;
                    }
                    pg[st] = pv;
                }
                const int xcol = DI + static_cast<int>(h) * D + 16 * hw + li;
                float vx[2][4];
#pragma unroll
                for (int st = 0; st < 2; ++st)
#pragma unroll
                    for (int v = 0; v < 4; ++v) vx[st][v] = proj_s[(16 * st + 4 * grp + v) * pp + xcol];
                f32x4_t Y = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int st = 0; st < 2; ++st)
#pragma unroll
                    for (int v = 0; v < 4; ++v) Y = __builtin_amdgcn_mfma_f32_16x16x4f32(pg[st][v], vx[st][v], Y, 0, 0, 0);
                const float skip = p.s.skip[h];
                float o[4];
#pragma unroll
                for (int v = 0; v < 4; ++v) {
                    const float y = fmaf(skip, vx[1][v], Y[v]);
                    o[v] = static_cast<float>(static_cast<double>(y) * lg[(hw * 4 + v) * 64 + lane]);
                }
                float* ocol = p.s.out + b * L * DI + h * D + 16 * hw + li;
                if (L == C) {
#pragma unroll
                    for (int v = 0; v < 4; ++v) store_off32(ocol, static_cast<unsigned>((16 + 4 * grp + v) * DI), o[v]);
                } else {
#pragma unroll
                    for (int v = 0; v < 4; ++v)
                        if (16 + 4 * grp + v < L) store_off32(ocol, static_cast<unsigned>((16 + 4 * grp + v) * DI), o[v]);
                }
            }
            return;
        }
    }
    scan_head<C, NT, DT, true, Hooks, false, HELP>(a, sh, b, h, 0, hooks);
}

// Geometries of the block kernel: (d_state, headdim, the in_proj's 32-wide k
// steps, the RMSNorm group size); false where none is built. The k steps
// follow the one-wave-per-tile linear's choice (2 up to K = 64, 4 up to 128,
// 8 up to 256), so the tiles run the same instructions.
bool launch_block_scan(const BlockArgs& p, int64_t N, int64_t D, int64_t gs, hipStream_t stream) {
    const int ksi = p.dm <= 64 ? 2 : (p.dm <= 128 ? 4 : 8);
    const size_t lds = sizeof(float) * 32 * static_cast<size_t>((p.W + 15) / 16 * 16 + 4);
    if (lds > 64 * 1024) return false;
    const dim3 grid(static_cast<unsigned>(p.s.B * p.s.H));
    // Column tiles a head reads: its z and x columns, the B/C rows, dt/A/trap/angles.
    const int64_t DI = p.s.H * D;
    const int64_t ncol = 2 * (D / 16) + (p.W - 2 * DI + 15) / 16;
#define MLK_BLOCK(NV, DV, KSIV, GSV, NCTV)                                                                       \
    if (N == NV && D == DV && ksi == KSIV && gs == GSV && ncol <= NCTV) {                                         \
        const bool all_live = p.dm == 32 * KSIV,                                                                 \
                   help = p.s.L <= 32 && p.s.G * NV == 16 && 3 * p.s.H + p.s.R <= 16 && ncol == NCTV;            \
        if (all_live && help) {                                                                                  \
            hipLaunchKernelGGL((mamba3_block_scan_kernel<NV / 16, DV / 16, KSIV, GSV, NCTV, true, true>), grid,   \
                               dim3(8 * DV), lds, stream, p);                                                     \
        } else if (all_live) {                                                                                   \
            hipLaunchKernelGGL((mamba3_block_scan_kernel<NV / 16, DV / 16, KSIV, GSV, NCTV, true, false>), grid,  \
                               dim3(4 * DV), lds, stream, p);                                                     \
        } else if (help) {                                                                                       \
            hipLaunchKernelGGL((mamba3_block_scan_kernel<NV / 16, DV / 16, KSIV, GSV, NCTV, false, true>), grid,  \
                               dim3(8 * DV), lds, stream, p);                                                     \
        } else {                                                                                                 \
            hipLaunchKernelGGL((mamba3_block_scan_kernel<NV / 16, DV / 16, KSIV, GSV, NCTV, false, false>), grid, \
                               dim3(4 * DV), lds, stream, p);                                                     \
        }                                                                                                        \
        return true;                                                                                             \
    }
    MLK_BLOCK(16, 32, 2, 8, 7)  // d_model up to 64 in groups of 8, d_state 16, heads of 32, 3H + R <= 16
#undef MLK_BLOCK
    return false;
}

template <int C>
bool launch_rec_chunk(const RecArgs& a, hipStream_t stream) {
    const int NT = static_cast<int>(a.N / 16), DT = static_cast<int>(a.D / 16);
    const dim3 grid(static_cast<unsigned>(a.B * a.H));
#define MLK_CHUNK(NTV, DTV)                                                                               \
    if (NT == NTV && DT == DTV) {                                                                         \
        hipLaunchKernelGGL((rec_chunk_kernel<C, NTV, DTV>), grid, dim3(64), 0, stream, a);              \
        return true;                                                                                      \
    }
    MLK_CHUNK(1, 2) MLK_CHUNK(1, 4) MLK_CHUNK(2, 2) MLK_CHUNK(2, 4) MLK_CHUNK(4, 2) MLK_CHUNK(4, 4)
#undef MLK_CHUNK
    return false;
}

mlk_status launch_rec(const RecArgs& a, hipStream_t stream) {
    if (a.B * a.L * a.H == 0 || a.D == 0) return MLK_OK;
    // Chunked scan on the matrix cores when there are at most 2048 (window,
    // head) pairs, i.e. at most two waves per SIMD: there the time-sequential
    // kernel's L dependent steps per wave leave the chip idle (measured
    // 0.058 vs 0.088 ms at 64 x 64 tokens, 8 heads, d_state 64). With more
    // pairs the sequential kernel fills the chip and is faster (1.17 vs 1.24
    // ms at 1024 x 256 tokens, 8 heads). d_state in {16, 32, 64}, headdim in
    // {32, 64}, 16-byte aligned q/k rows; MLK_MAMBA3_SCAN=sequential forces
    // the reference's own association.
    if (scan_mode() != ScanMode::kSequential && a.B * a.H <= 2048 && (a.N == 16 || a.N == 32 || a.N == 64) &&
        (a.D == 32 || a.D == 64) &&
        a.qs.t % 4 == 0 && a.qs.b % 4 == 0 && a.qs.h % 4 == 0 && a.ks.t % 4 == 0 && a.ks.b % 4 == 0 &&
        a.ks.h % 4 == 0 && aligned16(a.q) && aligned16(a.k)) {
        const bool ok = launch_rec_chunk<32>(a, stream);
        if (ok) return launch_status("mamba3 chunked recurrence");
    }
    const bool vec = a.D % 8 == 0;
    const bool pair = vec && a.D <= 32;
    const int64_t grid = a.B * a.H * ((a.D + (pair ? 31 : 63)) / (pair ? 32 : 64));
    const int N = static_cast<int>(a.N);
#define MLK_REC_LAUNCH(NM, EXACT, VEC, PAIR)                                                                     \
    hipLaunchKernelGGL((rec_kernel<NM, EXACT, VEC, PAIR>), dim3(grid), dim3(64), 0, stream, a.L, a.H, a.D, N, a.q, \
                       a.qs, a.k, a.ks, a.v, a.vs, a.gate, a.gs, a.gate_logits, a.alpha, a.beta, a.gamma, a.skip, \
                       a.out, a.os)
#define MLK_REC(NM, EXACT)                                                                                         \
    do {                                                                                                           \
        if (pair) {                                                                                                \
            MLK_REC_LAUNCH(NM, EXACT, true, true);                                                                 \
        } else if (vec) {                                                                                          \
            MLK_REC_LAUNCH(NM, EXACT, true, false);                                                                \
        } else {                                                                                                   \
            MLK_REC_LAUNCH(NM, EXACT, false, false);                                                               \
        }                                                                                                          \
        return launch_status("mamba3 recurrence");                                                                 \
    } while (0)
    switch (N) {
        case 16: MLK_REC(16, true);
        case 32: MLK_REC(32, true);
        case 64: MLK_REC(64, true);
        case 128: MLK_REC(128, true);
        default: break;
    }
    if (N <= 16) MLK_REC(16, false);
    if (N <= 64) MLK_REC(64, false);
    if (N <= 128) MLK_REC(128, false);
#undef MLK_REC
#undef MLK_REC_LAUNCH
    set_error("d_state above 128 is not supported by the GPU recurrence");
    return MLK_ERR_UNSUPPORTED;
}

// ---------------------------------------------------------------------------
// One-token step with carried state (no reference op; see mlk_hip.h)
// ---------------------------------------------------------------------------

struct StepArgs {
    int64_t S, N, G, H, D, R;
    const float* proj;  // [S, W] rows proj_ss apart
    int64_t proj_ss;
    const float* b_bias;
    const float* c_bias;
    const float* b_norm_w;
    const float* c_norm_w;
    float b_eps, c_eps;
    const float* dt_bias;
    const float* skip;
    float a_floor;
    float* ssm;     // [S, H, N, D]
    float* k_prev;  // [S, H, N]
    float* v_prev;  // [S, H, D]
    double* angle;  // [S, H, max(R, 1)]
    int started;    // 0 for the first token of a zero state: the beta term is dropped
    float* out;     // [S, H * D]
};

// One block of four waves per stream; wave w owns heads w, w+4, ... and its
// lanes are the headdim columns (D <= 64). Each wave issues the loads of its
// first head's [N, D] state before anything else, so the per-stream set-up
// below (B/C norms once per group, coefficients per head, the rotary phase
// of every (head, angle) pair in parallel) runs while the state streams in.
// Arithmetic per element is that of the sequence kernel.
constexpr int kStepThreads = 256;

template <int NM, bool VEC>
__global__ __launch_bounds__(kStepThreads) void step_kernel(StepArgs p) {
    extern __shared__ float lds[];
    const int64_t H = p.H, N = p.N, D = p.D, G = p.G, R = p.R;
    float* q_l = lds;            // [H][N] rotated q (from C)
    float* k_l = q_l + H * N;    // [H][N] rotated k (from B)
    float* kp_l = k_l + H * N;   // [H][N] previous k
    float* co = kp_l + H * N;    // [H][4] alpha, beta, gamma, dt
    float* sc = co + 4 * H;      // [2G] B scales, then C scales
    float* seg = sc + 2 * G;     // [2GN + 3H + R] the row's B | C | dt | A | trap | angles
    const int64_t s_idx = blockIdx.x;
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int64_t d_inner = H * D;
    const int64_t GN = G * N;
    const float* row = p.proj + s_idx * p.proj_ss;
    const float* b_raw = seg;
    const float* c_raw = b_raw + GN;
    const float* raw_dt = c_raw + GN;
    const float* raw_a = raw_dt + H;
    const float* raw_trap = raw_a + H;
    const float* raw_ang = raw_trap + H;
    const int started = p.started;

    // 1. State of this wave's first head: in flight from here on.
    float sv[NM];
    const int64_t h_first = wave;
    if (h_first < H && lane < D) {
        const float* st = p.ssm + ((s_idx * H + h_first) * N) * D + lane;
#pragma unroll
        for (int n = 0; n < NM; ++n) {
            if (n < N) sv[n] = st[static_cast<int64_t>(n) * D];
        }
    }

    // 2. Per-stream set-up, from the row slice staged in LDS.
    for (int64_t i = tid; i < 2 * GN + 3 * H + R; i += kStepThreads) seg[i] = row[2 * d_inner + i];
    if (started) {
        const float* kps = p.k_prev + s_idx * H * N;
        for (int64_t i = tid; i < H * N; i += kStepThreads) kp_l[i] = kps[i];
    }
    __syncthreads();
    if (tid < 2 * G) {
        const int64_t g = tid % G;
        sc[tid] = tid < G ? bc_norm_scale_lds(b_raw + g * N, N, p.b_eps)
                          : bc_norm_scale_lds(c_raw + g * N, N, p.c_eps);
    }
    if (tid >= 64 && tid < 64 + H) {
        const int64_t h = tid - 64;
        const float dt = softplus_f(raw_dt[h] + p.dt_bias[h]);
        const float a = -fmaxf(heavy_tail_f(raw_a[h]), p.a_floor);
        step_coefficients(a * dt, dt, raw_trap[h], &co[4 * h], &co[4 * h + 1], &co[4 * h + 2]);
        co[4 * h + 3] = dt;
    }
    __syncthreads();
    const int Ni = static_cast<int>(N), heads_per_group = static_cast<int>(H / G);
    for (int i = tid; i < H * N; i += kStepThreads) {
        const int h = i / Ni, n = i - h * Ni, g = h / heads_per_group;
        k_l[i] = (b_raw[g * N + n] * sc[g]) * p.b_norm_w[n] + p.b_bias[h * N + n];
        q_l[i] = (c_raw[g * N + n] * sc[G + g]) * p.c_norm_w[n] + p.c_bias[h * N + n];
    }
    __syncthreads();
    const int64_t Rw = R > 0 ? R : 1;
    const int Ri = static_cast<int>(R);
    for (int i = tid; i < H * R; i += kStepThreads) {
        const int h = i / Ri, r = i - h * Ri;
        double* run = p.angle + (s_idx * H + h) * Rw + r;
        const double next = *run + static_cast<double>((tanhf_cr(raw_ang[r]) * kPiF) * co[4 * h + 3]);
        *run = next;
        const float cumulative = static_cast<float>(next);
        const float wraps = __fmul_rn(kTwoPiF, floorf(cumulative / kTwoPiF));
        double sd, cd;
        sincos_d(static_cast<double>(cumulative - wraps), &sd, &cd);
        const float sine = static_cast<float>(sd), cosine = static_cast<float>(cd);
        float* pairs[2] = {q_l + h * N + 2 * r, k_l + h * N + 2 * r};
#pragma unroll
        for (int w = 0; w < 2; ++w) {
            const float l = pairs[w][0], rr = pairs[w][1];
            pairs[w][0] = fmaf(l, cosine, -(rr * sine));
            pairs[w][1] = fmaf(l, sine, rr * cosine);
        }
    }
    __syncthreads();

    // 3. Update and read out each head of this wave.
    for (int64_t h = wave; h < H; h += kStepThreads / 64) {
        const int d = lane;
        if (d >= D) continue;
        float* st = p.ssm + ((s_idx * H + h) * N) * D + d;
        if (h != h_first) {
#pragma unroll
            for (int n = 0; n < NM; ++n) {
                if (n < N) sv[n] = st[static_cast<int64_t>(n) * D];
            }
        }
        const float al = co[4 * h], be = co[4 * h + 1], ga = co[4 * h + 2];
        const float* x = row + d_inner + h * D;
        const float* z = row + h * D;
        float* vps = p.v_prev + (s_idx * H + h) * D;
        const float* qh = q_l + h * N;
        const float* kh = k_l + h * N;
        const float* kph = kp_l + h * N;
        const float v_cur = x[d];
        const float pv = started ? be * vps[d] : 0.0f;
        const float cv = ga * v_cur;
        float acc0 = 0.0f, acc1 = 0.0f;
#pragma unroll
        for (int n = 0; n < NM; ++n) {
            if (n < N) {
                const float kc = kh[n];
                const float kp = started ? kph[n] : kc;
                const float upd = (VEC || started) ? fmaf(kc, cv, fmaf(sv[n], al, kp * pv)) : fmaf(kc, cv, sv[n] * al);
                sv[n] = upd;
                if (VEC && (n & 1)) {
                    acc1 = fmaf(upd, qh[n], acc1);
                } else {
                    acc0 = fmaf(upd, qh[n], acc0);
                }
            }
        }
#pragma unroll
        for (int n = 0; n < NM; ++n) {
            // Non-temporal: the state is not read again this step, and leaving it
            // out of the caches keeps the projections' operands there (decode step
            // 4.30 -> 4.22 ms at 65536 streams, this kernel 1.87 -> 1.89 ms).
            if (n < N) __builtin_nontemporal_store(sv[n], st + static_cast<int64_t>(n) * D);
        }
        const float y = fmaf(p.skip[h], v_cur, VEC ? acc0 + acc1 : acc0);
        const double zz = static_cast<double>(z[d]);
        p.out[s_idx * d_inner + h * D + d] = static_cast<float>(static_cast<double>(y) * silu_d(zz));
        vps[d] = v_cur;
        float* kps = p.k_prev + (s_idx * H + h) * N;
        for (int64_t n = d; n < N; n += D) kps[n] = kh[n];
    }
}

}  // namespace
}  // namespace mlk

using namespace mlk;

extern "C" {

size_t mlk_mamba3_workspace_bytes(int64_t batch, int64_t length, int64_t nheads, int64_t d_state,
                                  int64_t num_rope_angles) {
    const int64_t blh = batch * length * nheads;
    const int64_t rw = num_rope_angles > 0 ? num_rope_angles : 1;
    return sizeof(float) * static_cast<size_t>(2 * blh * d_state + 3 * blh + blh * rw);
}

}  // extern "C"

namespace mlk {
namespace {

// mamba3_siso_recurrent with the (alpha, beta, gamma) coefficients in
// `coef` (3 * B * L * H floats): coef_kernel fills all of it before the
// recurrence reads it, so nothing in it needs clearing.
mlk_status siso_recurrent(const float* q, const int64_t* q_strides, const float* k, const int64_t* k_strides,
                          const float* v, const int64_t* v_strides, const float* gate, const int64_t* gate_strides,
                          const float* adt, const int64_t* adt_strides, const float* dt, const int64_t* dt_strides,
                          const float* trap_logit, const int64_t* trap_strides, const float* skip, int64_t batch,
                          int64_t length, int64_t heads, int64_t d_state, int64_t headdim, float* out, float* coef,
                          hipStream_t stream) {
    const int64_t blh = batch * length * heads;
    float* alpha = coef;
    float* beta = alpha + blh;
    float* gamma = beta + blh;
    auto s3 = [](const int64_t* x) { return Strides3{x[0], x[1], x[2]}; };
    MLK_CHECK(blh < (int64_t{1} << 31), "too many tokens x heads for one launch");
    hipLaunchKernelGGL(coef_kernel, dim3(ceil_div(blh, 256)), dim3(256), 0, stream, batch, length, heads, adt,
                       s3(adt_strides), dt, s3(dt_strides), trap_logit, s3(trap_strides), alpha, beta, gamma);
    const mlk_status st = launch_status("mamba3 coefficients");
    if (st != MLK_OK) return st;
    RecArgs a{};
    a.B = batch;
    a.L = length;
    a.H = heads;
    a.N = d_state;
    a.D = headdim;
    a.q = q;
    a.qs = s3(q_strides);
    a.k = k;
    a.ks = s3(k_strides);
    a.v = v;
    a.vs = s3(v_strides);
    a.gate = gate;
    a.gs = s3(gate_strides);
    a.gate_logits = 0;
    a.alpha = alpha;
    a.beta = beta;
    a.gamma = gamma;
    a.skip = skip;
    a.out = out;
    a.os = {length * heads * headdim, heads * headdim, headdim};
    return launch_rec(a, stream);
}

// Device memory of mlk_mamba3_siso_recurrent_noalloc: a file-scope array each
// GPU holds from module load to process end. Host code never uses the
// array's name as an address (on the host it is only a stand-in for the
// symbol); it uses the device address hipGetSymbolAddress returns, looked up
// once per device with that device current.
constexpr size_t kNoallocScratchBytes = MLK_NOALLOC_SCRATCH_BYTES;
__device__ __align__(256) unsigned char scratch[kNoallocScratchBytes];

constexpr int kMaxDevices = 64;
// g_scratch_mutex guards the per-device table and is held across each call's
// enqueue (wait, launches, record), so the calls' order on the array is the
// order in which they took the lock, whatever host thread or stream made them.
// g_scratch_done[device] is recorded on the calling stream after each use of
// that device's array, and the next call's stream waits on it first.
std::mutex g_scratch_mutex;
void* g_scratch_ptr[kMaxDevices] = {};
hipEvent_t g_scratch_done[kMaxDevices] = {};
bool g_scratch_recorded[kMaxDevices] = {};

// Looks the array's device address up (once per device, with that device
// current) and creates the device's event. The caller holds g_scratch_mutex.
mlk_status scratch_for_current_device(int* device_out) {
    int device = -1;
    hipError_t err = hipGetDevice(&device);
    if (err != hipSuccess) {
        set_error(std::string("mamba3_siso_recurrent_noalloc: hipGetDevice: ") + hipGetErrorString(err));
        return MLK_ERR_RUNTIME;
    }
    if (device < 0 || device >= kMaxDevices) {
        set_error("mamba3_siso_recurrent_noalloc: device index beyond the library's table");
        return MLK_ERR_UNSUPPORTED;
    }
    if (g_scratch_ptr[device] == nullptr) {
        void* found = nullptr;
        err = hipGetSymbolAddress(&found, HIP_SYMBOL(scratch));
        if (err != hipSuccess || found == nullptr) {
            set_error(std::string("mamba3_siso_recurrent_noalloc: hipGetSymbolAddress: ") + hipGetErrorString(err));
            return MLK_ERR_RUNTIME;
        }
        hipEvent_t done = nullptr;
        err = hipEventCreateWithFlags(&done, hipEventDisableTiming);
        if (err != hipSuccess) {
            set_error(std::string("mamba3_siso_recurrent_noalloc: hipEventCreateWithFlags: ") +
                      hipGetErrorString(err));
            return MLK_ERR_RUNTIME;
        }
        g_scratch_done[device] = done;
        g_scratch_ptr[device] = found;
    }
    *device_out = device;
    return MLK_OK;
}

}  // namespace
}  // namespace mlk

extern "C" {

mlk_status mlk_mamba3_siso_recurrent(const float* q, const int64_t* q_strides, const float* k,
                                     const int64_t* k_strides, const float* v, const int64_t* v_strides,
                                     const float* gate, const int64_t* gate_strides, const float* adt,
                                     const int64_t* adt_strides, const float* dt, const int64_t* dt_strides,
                                     const float* trap_logit, const int64_t* trap_strides, const float* skip,
                                     int64_t batch, int64_t length, int64_t heads, int64_t d_state,
                                     int64_t headdim, float* out, void* workspace, size_t workspace_bytes,
                                     mlk_stream_t stream) {
    MLK_CHECK(batch >= 0 && length >= 0 && heads >= 0 && d_state >= 0 && headdim >= 0, "q/k must be [B,L,H,N]");
    const int64_t blh = batch * length * heads;
    MLK_CHECK(workspace_bytes >= sizeof(float) * static_cast<size_t>(3 * blh), "workspace too small");
    if (blh == 0 || headdim == 0) return MLK_OK;
    MLK_CHECK(q && k && v && gate && adt && dt && trap_logit && skip && out && workspace, "null tensor pointer");
    MLK_CHECK(q_strides && k_strides && v_strides && gate_strides && adt_strides && dt_strides && trap_strides,
              "null stride array");
    return siso_recurrent(q, q_strides, k, k_strides, v, v_strides, gate, gate_strides, adt, adt_strides, dt,
                          dt_strides, trap_logit, trap_strides, skip, batch, length, heads, d_state, headdim, out,
                          static_cast<float*>(workspace), reinterpret_cast<hipStream_t>(stream));
}

mlk_status mlk_mamba3_siso_recurrent_noalloc(const float* q, const int64_t* q_strides, const float* k,
                                             const int64_t* k_strides, const float* v, const int64_t* v_strides,
                                             const float* gate, const int64_t* gate_strides, const float* adt,
                                             const int64_t* adt_strides, const float* dt, const int64_t* dt_strides,
                                             const float* trap_logit, const int64_t* trap_strides, const float* skip,
                                             int64_t batch, int64_t length, int64_t heads, int64_t d_state,
                                             int64_t headdim, float* out, mlk_stream_t stream) {
    MLK_CHECK(batch >= 0 && length >= 0 && heads >= 0 && d_state >= 0 && headdim >= 0, "q/k must be [B,L,H,N]");
    const int64_t blh = batch * length * heads;
    if (blh == 0 || headdim == 0) return MLK_OK;
    if (static_cast<uint64_t>(blh) > kNoallocScratchBytes / (3 * sizeof(float))) {
        set_error("mamba3_siso_recurrent_noalloc: batch * length * heads = " + std::to_string(blh) +
                  " exceeds the static scratch (" + std::to_string(kNoallocScratchBytes / (3 * sizeof(float))) +
                  " at most); use mlk_mamba3_siso_recurrent with a workspace");
        return MLK_ERR_INVALID_ARGUMENT;
    }
    MLK_CHECK(q && k && v && gate && adt && dt && trap_logit && skip && out, "null tensor pointer");
    MLK_CHECK(q_strides && k_strides && v_strides && gate_strides && adt_strides && dt_strides && trap_strides,
              "null stride array");
    const hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    // Outside capture the call's stream waits for the previous use of the array
    // on any stream and marks its own use. Under capture the graph's own order
    // holds: an event recorded outside a capture cannot be waited on inside it.
    hipStreamCaptureStatus capture = hipStreamCaptureStatusNone;
    hipError_t err = hipStreamIsCapturing(s, &capture);
    if (err != hipSuccess) {
        set_error(std::string("mamba3_siso_recurrent_noalloc: hipStreamIsCapturing: ") + hipGetErrorString(err));
        return MLK_ERR_RUNTIME;
    }
    const bool eager = capture == hipStreamCaptureStatusNone;
    std::lock_guard<std::mutex> lock(g_scratch_mutex);
    int device = -1;
    if (hipGetDevice(&device) == hipSuccess && device >= 0 && device < kMaxDevices && !eager &&
        g_scratch_ptr[device] == nullptr) {
        set_error("mamba3_siso_recurrent_noalloc: the first call on a device must be made outside graph capture");
        return MLK_ERR_INVALID_ARGUMENT;
    }
    const mlk_status st = scratch_for_current_device(&device);
    if (st != MLK_OK) return st;
    if (eager && g_scratch_recorded[device]) {
        err = hipStreamWaitEvent(s, g_scratch_done[device], 0);
        if (err != hipSuccess) {
            set_error(std::string("mamba3_siso_recurrent_noalloc: hipStreamWaitEvent: ") + hipGetErrorString(err));
            return MLK_ERR_RUNTIME;
        }
    }
    const mlk_status run = siso_recurrent(q, q_strides, k, k_strides, v, v_strides, gate, gate_strides, adt,
                                          adt_strides, dt, dt_strides, trap_logit, trap_strides, skip, batch, length,
                                          heads, d_state, headdim, out, static_cast<float*>(g_scratch_ptr[device]), s);
    if (run != MLK_OK || !eager) return run;
    err = hipEventRecord(g_scratch_done[device], s);
    if (err != hipSuccess) {
        set_error(std::string("mamba3_siso_recurrent_noalloc: hipEventRecord: ") + hipGetErrorString(err));
        return MLK_ERR_RUNTIME;
    }
    g_scratch_recorded[device] = true;
    return MLK_OK;
}

mlk_status mlk_mamba3_siso_forward(const float* projected, int64_t batch, int64_t length, int64_t width,
                                   int64_t proj_batch_stride, int64_t proj_token_stride, const float* gate,
                                   int64_t gate_batch_stride, int64_t gate_token_stride, const float* b_bias,
                                   const float* c_bias, const float* b_norm_w, const float* c_norm_w,
                                   const float* dt_bias, const float* skip, int64_t d_state, int64_t ngroups,
                                   int64_t nheads, int64_t headdim, int64_t num_rope_angles, double b_eps,
                                   double c_eps, double a_floor, float* out, void* workspace,
                                   size_t workspace_bytes, mlk_stream_t stream) {
    MLK_CHECK(d_state > 0 && ngroups > 0 && nheads > 0 && headdim > 0, "invalid Mamba-3 geometry");
    MLK_CHECK(nheads % ngroups == 0, "nheads must be divisible by ngroups");
    MLK_CHECK(num_rope_angles >= 0 && 2 * num_rope_angles <= d_state, "num_rope_angles must fit in d_state");
    const int64_t d_inner = nheads * headdim;
    const int64_t expected = 2 * d_inner + 2 * ngroups * d_state + 3 * nheads + num_rope_angles;
    if (width != expected) {
        set_error("projected width " + std::to_string(width) + " does not match the Mamba-3 layout width " +
                  std::to_string(expected));
        return MLK_ERR_INVALID_ARGUMENT;
    }
    MLK_CHECK(workspace_bytes >= mlk_mamba3_workspace_bytes(batch, length, nheads, d_state, num_rope_angles),
              "workspace too small");
    const int64_t blh = batch * length * nheads;
    if (blh == 0) return MLK_OK;
    MLK_CHECK(projected && b_bias && c_bias && b_norm_w && c_norm_w && dt_bias && skip && out && workspace,
              "null tensor pointer");
    // The fused kernel addresses a chunk's 32 rows by 32-bit byte offsets from its first row (row strides
    // below 2^25 floats); other strides take the separate kernels.
    const bool narrow_rows = proj_token_stride < (int64_t{1} << 25) &&
                             (gate == nullptr || gate_token_stride < (int64_t{1} << 25));
    if (scan_mode() == ScanMode::kFused && (d_state == 16 || d_state == 32 || d_state == 64) &&
        (headdim == 16 || headdim == 32 || headdim == 64) && batch * nheads < (int64_t{1} << 31) && narrow_rows) {
        ScanArgs s{};
        s.proj = projected;
        s.sb = proj_batch_stride;
        s.st = proj_token_stride;
        s.B = batch;
        s.L = length;
        s.G = ngroups;
        s.H = nheads;
        s.R = num_rope_angles;
        s.b_bias = b_bias;
        s.c_bias = c_bias;
        s.b_norm_w = b_norm_w;
        s.c_norm_w = c_norm_w;
        s.b_eps = static_cast<float>(b_eps);
        s.c_eps = static_cast<float>(c_eps);
        s.dt_bias = dt_bias;
        s.a_floor = static_cast<float>(a_floor);
        s.skip = skip;
        if (gate == nullptr) {
            s.gate = projected;
            s.gsb = proj_batch_stride;
            s.gst = proj_token_stride;
            s.gate_logits = 1;
        } else {
            s.gate = gate;
            s.gsb = gate_batch_stride;
            s.gst = gate_token_stride;
            s.gate_logits = 0;
        }
        s.out = out;
        if (launch_scan_fused(s, d_state, headdim, stream)) return launch_status("mamba3 fused scan");
    }
    const int64_t rw = num_rope_angles > 0 ? num_rope_angles : 1;
    float* q = static_cast<float*>(workspace);
    float* k = q + blh * d_state;
    float* alpha = k + blh * d_state;
    float* beta = alpha + blh;
    float* gamma = beta + blh;
    float* term = gamma + blh;
    (void)rw;
    PrepArgs pa{};
    pa.proj = projected;
    pa.sb = proj_batch_stride;
    pa.st = proj_token_stride;
    pa.B = batch;
    pa.L = length;
    pa.N = d_state;
    pa.G = ngroups;
    pa.H = nheads;
    pa.D = headdim;
    pa.R = num_rope_angles;
    pa.b_bias = b_bias;
    pa.c_bias = c_bias;
    pa.b_norm_w = b_norm_w;
    pa.c_norm_w = c_norm_w;
    pa.b_eps = static_cast<float>(b_eps);
    pa.c_eps = static_cast<float>(c_eps);
    pa.dt_bias = dt_bias;
    pa.a_floor = static_cast<float>(a_floor);
    pa.q = q;
    pa.k = k;
    pa.alpha = alpha;
    pa.beta = beta;
    pa.gamma = gamma;
    pa.term = term;
    const int tpb = ceil_div(batch * length, 32) >= 1024 ? 32 : 8;
    const size_t prep_lds = prep_lds_bytes(tpb, d_state, ngroups, nheads, num_rope_angles);
    MLK_CHECK(prep_lds <= 64 * 1024, "Mamba-3 in_proj layout too wide for the GPU prep kernel");
    if (tpb == 32) {
        hipLaunchKernelGGL(prep_kernel<32>, dim3(ceil_div(batch * length, 32)), dim3(256), prep_lds, stream, pa);
    } else {
        hipLaunchKernelGGL(prep_kernel<8>, dim3(ceil_div(batch * length, 8)), dim3(256), prep_lds, stream, pa);
    }
    mlk_status st = launch_status("mamba3 prep");
    if (st != MLK_OK) return st;
    if (num_rope_angles > 0) {
        MLK_CHECK(num_rope_angles <= kRotateLds, "too many rotary angles for the GPU rotate kernel");
        hipLaunchKernelGGL(rotate_kernel, dim3(batch * nheads), dim3(256), 0, stream, batch, length, nheads,
                           d_state, num_rope_angles, term, q, k);
        st = launch_status("mamba3 rotate");
        if (st != MLK_OK) return st;
    }
    RecArgs a{};
    a.B = batch;
    a.L = length;
    a.H = nheads;
    a.N = d_state;
    a.D = headdim;
    a.q = q;
    a.qs = {length * nheads * d_state, nheads * d_state, d_state};
    a.k = k;
    a.ks = a.qs;
    a.v = projected + d_inner;
    a.vs = {proj_batch_stride, proj_token_stride, headdim};
    if (gate == nullptr) {
        a.gate = projected;
        a.gs = {proj_batch_stride, proj_token_stride, headdim};
        a.gate_logits = 1;
    } else {
        a.gate = gate;
        a.gs = {gate_batch_stride, gate_token_stride, headdim};
        a.gate_logits = 0;
    }
    a.alpha = alpha;
    a.beta = beta;
    a.gamma = gamma;
    a.skip = skip;
    a.out = out;
    a.os = {length * d_inner, d_inner, headdim};
    return launch_rec(a, stream);
}

mlk_status mlk_mamba3_siso_step(const float* projected, int64_t streams, int64_t proj_stride, const float* b_bias,
                                const float* c_bias, const float* b_norm_w, const float* c_norm_w,
                                const float* dt_bias, const float* skip, int64_t d_state, int64_t ngroups,
                                int64_t nheads, int64_t headdim, int64_t num_rope_angles, double b_eps, double c_eps,
                                double a_floor, float* ssm_state, float* k_state, float* v_state,
                                double* angle_state, int started, float* out, mlk_stream_t stream) {
    MLK_CHECK(d_state > 0 && ngroups > 0 && nheads > 0 && headdim > 0, "invalid Mamba-3 geometry");
    MLK_CHECK(nheads % ngroups == 0, "nheads must be divisible by ngroups");
    MLK_CHECK(num_rope_angles >= 0 && 2 * num_rope_angles <= d_state, "num_rope_angles must fit in d_state");
    MLK_CHECK(headdim <= 64, "the GPU step handles headdim <= 64");
    MLK_CHECK(d_state <= 128, "d_state above 128 is not supported by the GPU step");
    if (streams == 0) return MLK_OK;
    MLK_CHECK(projected && b_bias && c_bias && b_norm_w && c_norm_w && dt_bias && skip && ssm_state && k_state &&
                  v_state && angle_state && out,
              "null tensor pointer");
    StepArgs p{};
    p.S = streams;
    p.N = d_state;
    p.G = ngroups;
    p.H = nheads;
    p.D = headdim;
    p.R = num_rope_angles;
    p.proj = projected;
    p.proj_ss = proj_stride;
    p.b_bias = b_bias;
    p.c_bias = c_bias;
    p.b_norm_w = b_norm_w;
    p.c_norm_w = c_norm_w;
    p.b_eps = static_cast<float>(b_eps);
    p.c_eps = static_cast<float>(c_eps);
    p.dt_bias = dt_bias;
    p.skip = skip;
    p.a_floor = static_cast<float>(a_floor);
    p.ssm = ssm_state;
    p.k_prev = k_state;
    p.v_prev = v_state;
    p.angle = angle_state;
    p.started = started;
    p.out = out;
    const bool vec = headdim % 8 == 0;
    const size_t lds_bytes = sizeof(float) * static_cast<size_t>(3 * nheads * d_state + 4 * nheads + 2 * ngroups +
                                                                 2 * ngroups * d_state + 3 * nheads + num_rope_angles);
    MLK_CHECK(lds_bytes <= 64 * 1024, "too many heads x d_state for the GPU step");
    MLK_CHECK(streams <= 0x7fffffff, "too many streams for one launch");
    const dim3 grid(static_cast<unsigned>(streams));
#define MLK_STEP(NM)                                                                                         \
    do {                                                                                                     \
        if (vec) {                                                                                           \
            hipLaunchKernelGGL((step_kernel<NM, true>), grid, dim3(kStepThreads), lds_bytes, stream, p);     \
        } else {                                                                                             \
            hipLaunchKernelGGL((step_kernel<NM, false>), grid, dim3(kStepThreads), lds_bytes, stream, p);    \
        }                                                                                                    \
        return launch_status("mamba3 step");                                                                 \
    } while (0)
    if (d_state <= 16) MLK_STEP(16);
    if (d_state <= 64) MLK_STEP(64);
    MLK_STEP(128);
#undef MLK_STEP
}

mlk_status mlk_rms_norm_mamba3_forward(const float* x, int64_t batch, int64_t length, int64_t d_model,
                                       int64_t x_batch_stride, int64_t x_token_stride, const float* norm_w,
                                       double norm_eps, int64_t norm_groups, const void* in_weight, int32_t in_dtype,
                                       const float* b_bias, const float* c_bias, const float* b_norm_w,
                                       const float* c_norm_w, const float* dt_bias, const float* skip,
                                       int64_t d_state, int64_t ngroups, int64_t nheads, int64_t headdim,
                                       int64_t num_rope_angles, double b_eps, double c_eps, double a_floor,
                                       float* out, mlk_stream_t stream) {
    MLK_CHECK(batch >= 0 && length >= 0 && d_model > 0, "inputs must be [B,L,d_model]");
    MLK_CHECK(norm_groups > 0 && d_model % norm_groups == 0, "groups must divide the normalised dimension");
    MLK_CHECK(d_state > 0 && ngroups > 0 && nheads > 0 && headdim > 0, "invalid Mamba-3 geometry");
    MLK_CHECK(nheads % ngroups == 0, "nheads must be divisible by ngroups");
    MLK_CHECK(num_rope_angles >= 0 && 2 * num_rope_angles <= d_state, "num_rope_angles must fit in d_state");
    MLK_CHECK(x_token_stride >= d_model, "inputs must be [B,L,d_model] with a dense last dimension");
    const int64_t width = 2 * nheads * headdim + 2 * ngroups * d_state + 3 * nheads + num_rope_angles;
    const int64_t gs = d_model / norm_groups;
    const bool vec = aligned16(x) && x_token_stride % 4 == 0 && x_batch_stride % 4 == 0 && aligned16(norm_w) &&
                     aligned16(in_weight) && d_model % 8 == 0;
    const bool built = d_state == 16 && headdim == 32 && gs == 8 && d_model <= 64 &&
                       sizeof(float) * 32 * static_cast<size_t>((width + 15) / 16 * 16 + 4) <= 64 * 1024;
    if (!vec || !built || in_dtype != MLK_DTYPE_F32 || ngroups != 1 || scan_mode() != ScanMode::kFused ||
        batch * nheads >= (int64_t{1} << 31)) {
        set_error("rms_norm_mamba3_forward: geometry without the fused kernel (use rms_norm_linear, then "
                  "mamba3_siso_forward)");
        return MLK_ERR_UNSUPPORTED;
    }
    if (batch * length == 0) return MLK_OK;
    MLK_CHECK(x && norm_w && in_weight && b_bias && c_bias && b_norm_w && c_norm_w && dt_bias && skip && out,
              "null tensor pointer");
    BlockArgs p{};
    p.x = x;
    p.x_bs = x_batch_stride;
    p.x_ts = x_token_stride;
    p.dm = d_model;
    p.W = width;
    p.norm_w = norm_w;
    p.norm_eps = static_cast<double>(static_cast<float>(norm_eps));
    p.in_w = static_cast<const float*>(in_weight);
    ScanArgs& s = p.s;
    s.B = batch;
    s.L = length;
    s.G = ngroups;
    s.H = nheads;
    s.R = num_rope_angles;
    s.b_bias = b_bias;
    s.c_bias = c_bias;
    s.b_norm_w = b_norm_w;
    s.c_norm_w = c_norm_w;
    s.b_eps = static_cast<float>(b_eps);
    s.c_eps = static_cast<float>(c_eps);
    s.dt_bias = dt_bias;
    s.a_floor = static_cast<float>(a_floor);
    s.skip = skip;
    s.out = out;
    if (!launch_block_scan(p, d_state, headdim, gs, reinterpret_cast<hipStream_t>(stream))) {
        set_error("rms_norm_mamba3_forward: geometry without the fused kernel (use rms_norm_linear, then "
                  "mamba3_siso_forward)");
        return MLK_ERR_UNSUPPORTED;
    }
    return launch_status("rms_norm_mamba3_forward");
}

}  // extern "C"
