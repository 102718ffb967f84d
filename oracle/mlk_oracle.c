/*
 * CPU oracle for the RDT4quant fused-forward path: a plain-C restatement of
 * the reference's CPU kernels (rdt4quant_cpu/montlok_{types,kernel,mhc,layers}.h)
 * and of the composite ops its PyTorch glue builds from them
 * (rdt4quant_cpu/montlok.cpp).
 *
 * TEST INFRASTRUCTURE ONLY. Only tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py may load this library, and only as the checker
 * or the timed CPU baseline. The product path (montlok.rdt on the GPU) never
 * calls it.
 *
 * Rounding contract. The reference is compiled with -ffp-contract=fast on an
 * FMA machine, so GCC fuses some multiply-adds. This file is compiled with
 * -ffp-contract=off and spells every fused operation out as fma()/fmaf(), so
 * the association is explicit. Where the reference's vector code keeps
 * several partial sums (4 double lanes, 2 vectors of 4, even/odd state rows)
 * the same partition is used here in scalar code. With that, every function
 * below reproduces the reference bit for bit, except where the reference uses
 * its own polynomial exp/sincos (gate silu, Mamba rotary sin/cos, SwiGLU):
 * those use libm here and agree to the last float ulp on all but a small
 * fraction of elements.
 *
 * Pins (tests/test_oracle.py): golden vectors written by the compiled
 * reference (tests/golden/), closed forms and invariants of each kernel, and
 * an fp64 brute force of the recurrence and of attention.
 *
 * GEMM and attention: the reference calls torch/oneDNN for these
 * (montlok.cpp:67-91, :1207-1208). orc_linear / orc_sdpa accumulate in double
 * and round once; they are pinned against torch's CPU routines in float64.
 */

#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#define MLK_PI_F 3.14159265358979323846f     /* montlok_types.h:54 */
#define MLK_TWO_PI_F 6.28318530717958647692f /* montlok_types.h:55 */

/* ------------------------------------------------------------------------ */
/* Scalar helpers: montlok_types.h:57-93                                      */
/* ------------------------------------------------------------------------ */

/* torch softplus(beta=1, threshold=20), montlok_types.h:58-60 */
static float softplus_f(float x) { return x > 20.0f ? x : log1pf(expf(x)); }

/* montlok_types.h:62-64 */
static float sigmoid_f(float x) { return 1.0f / (1.0f + expf(-x)); }

/* montlok_types.h:67-71 */
static float heavy_tail_f(float x) {
    const float negative = x < 0.0f ? x : 0.0f;
    const float positive = x > 0.0f ? x : 0.0f;
    return positive + 1.0f / (1.0f - negative);
}

/* montlok_types.h:89-93 */
static void step_coefficients(float adt, float dt, float trap_logit, float* alpha, float* beta, float* gamma) {
    const float a = expf(adt);
    const float trap = sigmoid_f(trap_logit);
    *alpha = a;
    *beta = ((1.0f - trap) * dt) * a;
    *gamma = trap * dt;
}

/* montlok_mhc.h:23-25 */
static double sigmoid_d(double x) { return 1.0 / (1.0 + exp(-x)); }

/* silu(z) * y in double, rounded once: montlok_kernel.h:169-189 (the
 * reference evaluates exp with its own polynomial, here libm). */
static float gate_silu(float y, float z) {
    const double zd = (double)z;
    return (float)((double)y * (zd / (1.0 + exp(-zd))));
}

/* Sum of squares of fp32 values in double with the reference's partition:
 * two 4-lane accumulators over 8-element steps, hsum ((a0+a1)+(a2+a3)) of
 * their lane sums, then a scalar tail (montlok_layers.h:31-49). */
static double sumsq_f8(const float* x, int64_t count) {
    double acc0[4] = {0, 0, 0, 0};
    double acc1[4] = {0, 0, 0, 0};
    int64_t k = 0;
    for (; k + 8 <= count; k += 8) {
        for (int l = 0; l < 4; ++l) {
            const double a = (double)x[k + l];
            const double b = (double)x[k + 4 + l];
            acc0[l] = fma(a, a, acc0[l]);
            acc1[l] = fma(b, b, acc1[l]);
        }
    }
    double t[4];
    for (int l = 0; l < 4; ++l) {
        t[l] = acc0[l] + acc1[l];
    }
    double sum = (t[0] + t[1]) + (t[2] + t[3]);
    for (; k < count; ++k) {
        const double v = (double)x[k];
        sum = fma(v, v, sum);
    }
    return sum;
}

/* ------------------------------------------------------------------------ */
/* RMSNorm / GroupedRMSNorm: montlok_layers.h:20-65, op montlok.cpp:915-938   */
/* ------------------------------------------------------------------------ */

static void rms_norm_row(const float* xr, const float* w, double eps, int64_t dim, int64_t groups, float* outr) {
    const int64_t gs = dim / groups;
    for (int64_t g = 0; g < groups; ++g) {
        const float* xg = xr + g * gs;
        const float* wg = w + g * gs;
        float* og = outr + g * gs;
        const double sumsq = sumsq_f8(xg, gs);
        const double scale = 1.0 / sqrt(sumsq / (double)gs + eps);
        for (int64_t k = 0; k < gs; ++k) {
            og[k] = (float)(((double)xg[k] * scale) * (double)wg[k]);
        }
    }
}

/* eps arrives as the Python float and is cast through float32 (montlok.cpp:932). */
void orc_rms_norm(const float* x, int64_t row_stride, const float* w, double eps, int64_t dim, int64_t groups,
                  int64_t rows, float* out) {
    const double eps_f = (double)(float)eps;
    for (int64_t row = 0; row < rows; ++row) {
        rms_norm_row(x + row * row_stride, w, eps_f, dim, groups, out + row * dim);
    }
}

/* residual = left + right in fp32, then RMSNorm: montlok_layers.h:71-90 */
void orc_add_rms_norm(const float* left, const float* right, const float* w, double eps, int64_t dim,
                      int64_t groups, int64_t rows, float* residual, float* normalized) {
    const double eps_f = (double)(float)eps;
    for (int64_t row = 0; row < rows; ++row) {
        float* res = residual + row * dim;
        for (int64_t k = 0; k < dim; ++k) {
            res[k] = left[row * dim + k] + right[row * dim + k];
        }
        rms_norm_row(res, w, eps_f, dim, groups, normalized + row * dim);
    }
}

/* ------------------------------------------------------------------------ */
/* LayerNorm: montlok_layers.h:117-184, op montlok.cpp:1057-1082             */
/* ------------------------------------------------------------------------ */

void orc_layer_norm(const float* x, int64_t row_stride, const float* w, const float* bias, double eps, int64_t dim,
                    int64_t rows, float* out) {
    const double eps_f = (double)(float)eps;
    const double inv_dim = 1.0 / (double)dim;
    for (int64_t row = 0; row < rows; ++row) {
        const float* xr = x + row * row_stride;
        float* outr = out + row * dim;
        double acc0[4] = {0, 0, 0, 0}, acc1[4] = {0, 0, 0, 0};
        int64_t k = 0;
        for (; k + 8 <= dim; k += 8) {
            for (int l = 0; l < 4; ++l) {
                acc0[l] += (double)xr[k + l];
                acc1[l] += (double)xr[k + 4 + l];
            }
        }
        double t[4];
        for (int l = 0; l < 4; ++l) t[l] = acc0[l] + acc1[l];
        double sum = (t[0] + t[1]) + (t[2] + t[3]);
        for (; k < dim; ++k) sum += (double)xr[k];
        const double mean = sum * inv_dim;

        for (int l = 0; l < 4; ++l) acc0[l] = acc1[l] = 0.0;
        k = 0;
        for (; k + 8 <= dim; k += 8) {
            for (int l = 0; l < 4; ++l) {
                const double a = (double)xr[k + l] - mean;
                const double b = (double)xr[k + 4 + l] - mean;
                acc0[l] = fma(a, a, acc0[l]);
                acc1[l] = fma(b, b, acc1[l]);
            }
        }
        for (int l = 0; l < 4; ++l) t[l] = acc0[l] + acc1[l];
        double sumsq = (t[0] + t[1]) + (t[2] + t[3]);
        for (; k < dim; ++k) {
            const double a = (double)xr[k] - mean;
            sumsq = fma(a, a, sumsq);
        }
        const double rstd = 1.0 / sqrt(fma(sumsq, inv_dim, eps_f));
        for (k = 0; k < dim; ++k) {
            const double y = (((double)xr[k] - mean) * rstd) * (double)w[k];
            outr[k] = (float)(bias != NULL ? y + (double)bias[k] : y);
        }
    }
}

/* ------------------------------------------------------------------------ */
/* SwiGLU gate: montlok_layers.h:95-112, op montlok.cpp:942-963              */
/* ------------------------------------------------------------------------ */

void orc_swiglu(const float* x, int64_t row_stride, int64_t hidden, int64_t rows, float* out) {
    for (int64_t row = 0; row < rows; ++row) {
        const float* gate = x + row * row_stride;
        const float* up = gate + hidden;
        for (int64_t k = 0; k < hidden; ++k) {
            const double z = (double)gate[k];
            out[row * hidden + k] = (float)((z / (1.0 + exp(-z))) * (double)up[k]);
        }
    }
}

/* ------------------------------------------------------------------------ */
/* Mamba-3 SISO recurrence: montlok_kernel.h:251-457                         */
/* ------------------------------------------------------------------------ */

/* Per-token coefficients of mamba3_siso_recurrent (montlok.cpp:279-299). */
void orc_step_coefficients(const float* adt, const float* dt, const float* trap, int64_t count, float* alpha,
                           float* beta, float* gamma) {
    for (int64_t i = 0; i < count; ++i) {
        step_coefficients(adt[i], dt[i], trap[i], alpha + i, beta + i, gamma + i);
    }
}

/* Block width of the reference's vector path (montlok_types.h:141-152): 16
 * or 8 lanes when the headdim allows, else the scalar whole-head path. The
 * two paths differ only in how the q . state reduction is split: the vector
 * path keeps even and odd state rows in two accumulators
 * (montlok_kernel.h:300-322), the scalar path one (:391-401). */
static int siso_vector_path(int64_t D) { return D % 8 == 0; }

/* One (b, h) head over all time steps. Strides (elements) of the leading
 * [B, L, H] dimensions are given per tensor; the last dimension is dense.
 * alpha/beta/gamma are contiguous [B, L, H]. The state starts at zero. */
static void siso_head(int64_t L, int64_t H, int64_t N, int64_t D, const float* q_row, const int64_t* qs,
                      const float* k_row, const int64_t* ks, const float* v_row, const int64_t* vs,
                      const float* g_row, const int64_t* gs, int gate_logits, const float* ca, const float* cb,
                      const float* cg, float skip, float* o_row, const int64_t* os, float* state, float* acc0,
                      float* acc1) {
    const int vec = siso_vector_path(D);
    memset(state, 0, sizeof(float) * (size_t)(N * D));
    for (int64_t t = 0; t < L; ++t) {
        const float al = ca[t * H];
        const float be = cb[t * H];
        const float ga = cg[t * H];
        const float* k_prev = t > 0 ? k_row - ks[1] : k_row;
        const float* v_prev = t > 0 ? v_row - vs[1] : NULL;
        for (int64_t d = 0; d < D; ++d) {
            acc0[d] = 0.0f;
            acc1[d] = 0.0f;
        }
        for (int64_t n = 0; n < N; ++n) {
            float* s = state + n * D;
            const float kp = k_prev[n];
            const float kc = k_row[n];
            const float qn = q_row[n];
            /* Even rows feed acc0, odd rows acc1 on the vector path; the
             * scalar path has one accumulator. A trailing odd row of the
             * vector path goes to acc0 (montlok_kernel.h:323-334). */
            float* acc = (vec && (n & 1)) ? acc1 : acc0;
            for (int64_t d = 0; d < D; ++d) {
                const float pv = v_prev != NULL ? be * v_prev[d] : 0.0f;
                const float cv = ga * v_row[d];
                /* s * al + kp * pv + kc * cv, contracted as
                 * fma(kc, cv, fma(s, al, kp * pv)). */
                float updated;
                if (vec) {
                    updated = fmaf(kc, cv, fmaf(s[d], al, kp * pv));
                } else if (v_prev != NULL) {
                    updated = fmaf(kc, cv, fmaf(s[d], al, kp * pv));
                } else {
                    updated = fmaf(kc, cv, s[d] * al);
                }
                s[d] = updated;
                acc[d] = fmaf(updated, qn, acc[d]);
            }
        }
        for (int64_t d = 0; d < D; ++d) {
            const float sum = vec ? acc0[d] + acc1[d] : acc0[d];
            const float y = fmaf(skip, v_row[d], sum);
            o_row[d] = gate_logits ? gate_silu(y, g_row[d]) : y * g_row[d];
        }
        q_row += qs[1];
        k_row += ks[1];
        v_row += vs[1];
        g_row += gs[1];
        o_row += os[1];
    }
}

void orc_siso(int64_t B, int64_t L, int64_t H, int64_t N, int64_t D, const float* q, const int64_t* qs,
              const float* k, const int64_t* ks, const float* v, const int64_t* vs, const float* gate,
              const int64_t* gs, int gate_logits, const float* alpha, const float* beta, const float* gamma,
              const float* skip, float* out, const int64_t* os) {
    float* state = (float*)malloc(sizeof(float) * (size_t)(N * D + 2 * D));
    for (int64_t b = 0; b < B; ++b) {
        for (int64_t h = 0; h < H; ++h) {
            const int64_t c0 = b * L * H + h;
            siso_head(L, H, N, D, q + b * qs[0] + h * qs[2], qs, k + b * ks[0] + h * ks[2], ks,
                      v + b * vs[0] + h * vs[2], vs, gate + b * gs[0] + h * gs[2], gs, gate_logits, alpha + c0,
                      beta + c0, gamma + c0, skip[h], out + b * os[0] + h * os[2], os, state, state + N * D,
                      state + N * D + D);
        }
    }
    free(state);
}

/* ------------------------------------------------------------------------ */
/* Mamba-3 pre-processing, phases A/B/C: montlok_kernel.h:463-597            */
/* ------------------------------------------------------------------------ */

/* BCNorm, fp32 throughout (montlok_kernel.h:464-474). The sum of squares is
 * sequential. In the compiled reference (AVX2 variant) GCC vectorises the
 * squares of the first 4*floor(n/4) elements (8- then 4-float vectors, each
 * square rounded before the in-order add) and contracts the scalar remainder
 * into fma. (The reference's AVX-512 variant vectorises 8*floor(n/8); the two
 * differ by an ulp when n mod 8 >= 4. n = 16 and 64 agree.) */
static void bc_norm(const float* x, const float* w, float eps, int64_t n, float* out) {
    float ss = 0.0f;
    const int64_t body = n - n % 4;
    for (int64_t i = 0; i < body; ++i) ss = ss + x[i] * x[i];
    for (int64_t i = body; i < n; ++i) ss = fmaf(x[i], x[i], ss);
    const float scale = 1.0f / sqrtf(ss / (float)n + eps);
    for (int64_t i = 0; i < n; ++i) out[i] = (x[i] * scale) * w[i];
}

/* Phase A for one token (montlok_kernel.h:477-526). */
static void prep_token(const float* row, int64_t d_inner, int64_t N, int64_t G, int64_t H, int64_t R,
                       const float* b_bias, const float* c_bias, const float* b_norm_w, const float* c_norm_w,
                       float b_eps, float c_eps, const float* dt_bias, float a_floor, float* q_tok, float* k_tok,
                       float* alpha, float* beta, float* gamma, float* term, float* scratch) {
    const int64_t GN = G * N;
    const float* b_raw = row + 2 * d_inner;
    const float* c_raw = b_raw + GN;
    const float* raw_dt = c_raw + GN;
    const float* raw_a = raw_dt + H;
    const float* raw_trap = raw_a + H;
    const float* raw_angles = raw_trap + H;
    float* bn = scratch;
    float* cn = scratch + GN;
    float* angles = scratch + 2 * GN;
    for (int64_t g = 0; g < G; ++g) {
        bc_norm(b_raw + g * N, b_norm_w, b_eps, N, bn + g * N);
        bc_norm(c_raw + g * N, c_norm_w, c_eps, N, cn + g * N);
    }
    for (int64_t r = 0; r < R; ++r) angles[r] = tanhf(raw_angles[r]) * MLK_PI_F;
    const int64_t per_group = H / G;
    for (int64_t h = 0; h < H; ++h) {
        const int64_t g = h / per_group;
        for (int64_t n = 0; n < N; ++n) {
            k_tok[h * N + n] = bn[g * N + n] + b_bias[h * N + n];
            q_tok[h * N + n] = cn[g * N + n] + c_bias[h * N + n];
        }
        const float dt = softplus_f(raw_dt[h] + dt_bias[h]);
        const float ht = heavy_tail_f(raw_a[h]);
        const float a = -(ht > a_floor ? ht : a_floor);
        step_coefficients(a * dt, dt, raw_trap[h], alpha + h, beta + h, gamma + h);
        for (int64_t r = 0; r < R; ++r) term[h * R + r] = angles[r] * dt;
    }
}

/* Phase C rotation of one interleaved pair (montlok_kernel.h:564-569),
 * contracted as fma(l, c, -(r * s)) and fma(l, s, r * c). */
static void rotate_pair(float* pair, float sine, float cosine) {
    const float left = pair[0];
    const float right = pair[1];
    pair[0] = fmaf(left, cosine, -(right * sine));
    pair[1] = fmaf(left, sine, right * cosine);
}

/* Wrap of the cumulative angle into [0, 2pi) with the product rounded on its
 * own (montlok_kernel.h:584-588). */
static float wrap_angle(float cumulative) {
    volatile float wraps = MLK_TWO_PI_F * floorf(cumulative / MLK_TWO_PI_F);
    return cumulative - wraps;
}

/* All three phases (montlok.cpp:443-461). q, k: [B, L, H, N] contiguous;
 * alpha/beta/gamma [B, L, H]. The angle cumulative sum is carried in double
 * and rounded to float at each step (montlok_kernel.h:529-542). */
void orc_prep(int64_t B, int64_t L, const float* proj, int64_t proj_sb, int64_t proj_st, int64_t d_inner,
              int64_t N, int64_t G, int64_t H, int64_t R, const float* b_bias, const float* c_bias,
              const float* b_norm_w, const float* c_norm_w, double b_eps, double c_eps, const float* dt_bias,
              double a_floor, float* q, float* k, float* alpha, float* beta, float* gamma) {
    const int64_t Rw = R > 0 ? R : 1;
    float* term = (float*)malloc(sizeof(float) * (size_t)(B * L * H * Rw));
    float* scratch = (float*)malloc(sizeof(float) * (size_t)(2 * G * N + Rw));
    double* running = (double*)malloc(sizeof(double) * (size_t)(H * Rw));
    for (int64_t b = 0; b < B; ++b) {
        for (int64_t t = 0; t < L; ++t) {
            const int64_t tok = b * L + t;
            prep_token(proj + b * proj_sb + t * proj_st, d_inner, N, G, H, R, b_bias, c_bias, b_norm_w, c_norm_w,
                       (float)b_eps, (float)c_eps, dt_bias, (float)a_floor, q + tok * H * N, k + tok * H * N,
                       alpha + tok * H, beta + tok * H, gamma + tok * H, term + tok * H * Rw, scratch);
        }
    }
    if (R > 0) {
        for (int64_t b = 0; b < B; ++b) {
            for (int64_t i = 0; i < H * R; ++i) running[i] = 0.0;
            for (int64_t t = 0; t < L; ++t) {
                const int64_t tok = b * L + t;
                for (int64_t h = 0; h < H; ++h) {
                    float* qh = q + (tok * H + h) * N;
                    float* kh = k + (tok * H + h) * N;
                    for (int64_t r = 0; r < R; ++r) {
                        running[h * R + r] += (double)term[(tok * H + h) * Rw + r];
                        const float cumulative = (float)running[h * R + r];
                        const double angle = (double)wrap_angle(cumulative);
                        const float sine = (float)sin(angle);
                        const float cosine = (float)cos(angle);
                        rotate_pair(qh + 2 * r, sine, cosine);
                        rotate_pair(kh + 2 * r, sine, cosine);
                    }
                }
            }
        }
    }
    free(running);
    free(scratch);
    free(term);
}

/* mamba3_siso_forward with an empty gate (montlok.cpp:333-492): phases A-C,
 * then the recurrence with v and z read straight from the in_proj rows and
 * silu(z) evaluated in the kernel. out: [B, L, H*D] contiguous. */
void orc_mamba3_siso_forward(int64_t B, int64_t L, const float* proj, int64_t proj_sb, int64_t proj_st, int64_t N,
                             int64_t G, int64_t H, int64_t D, int64_t R, const float* b_bias, const float* c_bias,
                             const float* b_norm_w, const float* c_norm_w, double b_eps, double c_eps,
                             const float* dt_bias, const float* skip, double a_floor, float* out) {
    const int64_t d_inner = H * D;
    const int64_t BLH = B * L * H;
    float* q = (float*)malloc(sizeof(float) * (size_t)(BLH * N));
    float* k = (float*)malloc(sizeof(float) * (size_t)(BLH * N));
    float* coef = (float*)malloc(sizeof(float) * (size_t)(3 * BLH));
    orc_prep(B, L, proj, proj_sb, proj_st, d_inner, N, G, H, R, b_bias, c_bias, b_norm_w, c_norm_w, b_eps, c_eps,
             dt_bias, a_floor, q, k, coef, coef + BLH, coef + 2 * BLH);
    const int64_t qs[3] = {L * H * N, H * N, N};
    const int64_t vs[3] = {proj_sb, proj_st, D};
    const int64_t os[3] = {L * d_inner, d_inner, D};
    orc_siso(B, L, H, N, D, q, qs, k, qs, proj + d_inner, vs, proj, vs, 1, coef, coef + BLH, coef + 2 * BLH, skip,
             out, os);
    free(coef);
    free(k);
    free(q);
}

/* One recurrent step of the same layer for S independent streams with
 * carried state (no reference op: the state the sequence kernel keeps in
 * registers, made explicit). Per stream: ssm [H, N, D] fp32, k_prev [H, N],
 * v_prev [H, D], angle [H, R] double (the phase-B running sum), and `started`
 * (0 before the first token: the beta term is then dropped, as at t = 0 of
 * the sequence kernel). proj: [S, W] in_proj rows of the current token.
 * Stepping T times from a zero state reproduces orc_mamba3_siso_forward over
 * T tokens bit for bit. */
void orc_mamba3_step(int64_t S, const float* proj, int64_t proj_ss, int64_t N, int64_t G, int64_t H, int64_t D,
                     int64_t R, const float* b_bias, const float* c_bias, const float* b_norm_w,
                     const float* c_norm_w, double b_eps, double c_eps, const float* dt_bias, const float* skip,
                     double a_floor, float* ssm, float* k_prev, float* v_prev, double* angle, int started,
                     float* out) {
    const int64_t d_inner = H * D;
    const int64_t Rw = R > 0 ? R : 1;
    float* qk = (float*)malloc(sizeof(float) * (size_t)(2 * H * N + 3 * H + H * Rw + 2 * G * N + Rw));
    float* q = qk;
    float* k = q + H * N;
    float* ca = k + H * N;
    float* cb = ca + H;
    float* cg = cb + H;
    float* term = cg + H;
    float* scratch = term + H * Rw;
    float* acc0 = (float*)malloc(sizeof(float) * (size_t)(2 * D));
    float* acc1 = acc0 + D;
    const int vec = siso_vector_path(D);
    for (int64_t s = 0; s < S; ++s) {
        const float* row = proj + s * proj_ss;
        prep_token(row, d_inner, N, G, H, R, b_bias, c_bias, b_norm_w, c_norm_w, (float)b_eps, (float)c_eps,
                   dt_bias, (float)a_floor, q, k, ca, cb, cg, term, scratch);
        for (int64_t h = 0; h < H; ++h) {
            double* run = angle + (s * H + h) * Rw;
            for (int64_t r = 0; r < R; ++r) {
                run[r] += (double)term[h * Rw + r];
                const double a = (double)wrap_angle((float)run[r]);
                const float sine = (float)sin(a);
                const float cosine = (float)cos(a);
                rotate_pair(q + h * N + 2 * r, sine, cosine);
                rotate_pair(k + h * N + 2 * r, sine, cosine);
            }
        }
        const float* z = row;
        const float* x = row + d_inner;
        for (int64_t h = 0; h < H; ++h) {
            float* st = ssm + (s * H + h) * N * D;
            float* kp_s = k_prev + (s * H + h) * N;
            float* vp_s = v_prev + (s * H + h) * D;
            const float* kc_h = k + h * N;
            const float* q_h = q + h * N;
            const float* v_h = x + h * D;
            for (int64_t d = 0; d < D; ++d) acc0[d] = acc1[d] = 0.0f;
            for (int64_t n = 0; n < N; ++n) {
                float* srow = st + n * D;
                float* acc = (vec && (n & 1)) ? acc1 : acc0;
                for (int64_t d = 0; d < D; ++d) {
                    const float cv = cg[h] * v_h[d];
                    float updated;
                    if (started) {
                        const float pv = cb[h] * vp_s[d];
                        updated = fmaf(kc_h[n], cv, fmaf(srow[d], ca[h], kp_s[n] * pv));
                    } else if (vec) {
                        updated = fmaf(kc_h[n], cv, fmaf(srow[d], ca[h], kc_h[n] * 0.0f));
                    } else {
                        updated = fmaf(kc_h[n], cv, srow[d] * ca[h]);
                    }
                    srow[d] = updated;
                    acc[d] = fmaf(updated, q_h[n], acc[d]);
                }
            }
            for (int64_t d = 0; d < D; ++d) {
                const float sum = vec ? acc0[d] + acc1[d] : acc0[d];
                const float y = fmaf(skip[h], v_h[d], sum);
                out[s * d_inner + h * D + d] = gate_silu(y, z[h * D + d]);
                vp_s[d] = v_h[d];
            }
            for (int64_t n = 0; n < N; ++n) kp_s[n] = kc_h[n];
        }
    }
    free(acc0);
    free(qk);
}

/* orc_mamba3_step over `threads` contiguous ranges of the streams at once.
 * The streams are independent, so the result equals one call over all of
 * them; the split only serves the CPU baseline's multi-core timing. */
void orc_mamba3_step_threads(int threads, int64_t S, const float* proj, int64_t proj_ss, int64_t N, int64_t G,
                             int64_t H, int64_t D, int64_t R, const float* b_bias, const float* c_bias,
                             const float* b_norm_w, const float* c_norm_w, double b_eps, double c_eps,
                             const float* dt_bias, const float* skip, double a_floor, float* ssm, float* k_prev,
                             float* v_prev, double* angle, int started, float* out) {
    const int64_t Rw = R > 0 ? R : 1;
    if (threads < 1) threads = 1;
#pragma omp parallel for num_threads(threads) schedule(static, 1)
    for (int t = 0; t < threads; ++t) {
        const int64_t a = S * t / threads, b = S * (t + 1) / threads;
        if (b > a) {
            orc_mamba3_step(b - a, proj + a * proj_ss, proj_ss, N, G, H, D, R, b_bias, c_bias, b_norm_w, c_norm_w,
                            b_eps, c_eps, dt_bias, skip, a_floor, ssm + a * H * N * D, k_prev + a * H * N,
                            v_prev + a * H * D, angle + a * H * Rw, started, out + a * H * D);
        }
    }
}

/* ------------------------------------------------------------------------ */
/* mHC read side: montlok_mhc.h:23-322, op montlok.cpp:659-691               */
/* ------------------------------------------------------------------------ */

/* w . ref over d with four double lanes (i mod 4), hsum, scalar tail
 * (montlok_mhc.h:32-75). */
static double dot_lanes(const double* w, const double* ref, int64_t d) {
    double acc[4] = {0, 0, 0, 0};
    int64_t i = 0;
    for (; i + 4 <= d; i += 4) {
        for (int l = 0; l < 4; ++l) acc[l] = fma(w[i + l], ref[i + l], acc[l]);
    }
    double out = (acc[0] + acc[1]) + (acc[2] + acc[3]);
    for (; i < d; ++i) out = fma(w[i], ref[i], out);
    return out;
}

/* Linear-space Sinkhorn of one n x n matrix, max(iters, 1) rounds of row then
 * column normalisation (montlok_mhc.h:96-157). m holds logits on entry. */
static void sinkhorn(double* m, double* sums, int64_t n, int iters) {
    for (int64_t e = 0; e < n * n; ++e) m[e] = exp(m[e]);
    const int rounds = iters > 1 ? iters : 1;
    for (int it = 0; it < rounds; ++it) {
        for (int64_t i = 0; i < n; ++i) {
            double s = m[i * n];
            for (int64_t j = 1; j < n; ++j) s += m[i * n + j];
            const double inv = 1.0 / s;
            for (int64_t j = 0; j < n; ++j) m[i * n + j] *= inv;
        }
        for (int64_t j = 0; j < n; ++j) {
            double s = m[j];
            for (int64_t i = 1; i < n; ++i) s += m[i * n + j];
            sums[j] = 1.0 / s;
        }
        for (int64_t i = 0; i < n; ++i) {
            for (int64_t j = 0; j < n; ++j) m[i * n + j] *= sums[j];
        }
    }
}

/* In-place RMSNorm of one aggregate row (montlok_mhc.h:162-193). */
static void agg_norm_inplace(float* x, const float* w, double eps, int64_t d) {
    const double sumsq = sumsq_f8(x, d);
    const double scale = 1.0 / sqrt(sumsq / (double)d + eps);
    for (int64_t k = 0; k < d; ++k) x[k] = (float)(((double)x[k] * scale) * (double)w[k]);
}

/* One token of mhc_prepare_block (montlok_mhc.h:198-322). */
static void mhc_prepare_token(const float* streams, int64_t sd, const float* norm_w, const double* proj_w,
                              const float* pre_bias, const float* post_bias, const float* res_bias, double pre_alpha,
                              double post_alpha, double res_alpha, double eps, int64_t n, int64_t d, int iters,
                              const float* agg_norm_w, double agg_norm_eps, float* agg, float* pre, float* post,
                              float* res, double* scratch) {
    const int64_t rows = 2 * n + n * n;
    double* ref = scratch;
    double* logit = ref + d;
    double* mat = logit + rows;
    double* sums = mat + n * n;
    const double inv_n = 1.0 / (double)n;

    /* ref = RMSNorm(mean_i streams_i) in double; the squares go to four lanes
     * (k mod 4) over the 4-aligned part, then a scalar tail. */
    double sq[4] = {0, 0, 0, 0};
    int64_t k = 0;
    for (; k + 4 <= d; k += 4) {
        for (int l = 0; l < 4; ++l) {
            double m = (double)streams[k + l];
            for (int64_t i = 1; i < n; ++i) m += (double)streams[i * sd + k + l];
            m *= inv_n;
            ref[k + l] = m;
            sq[l] = fma(m, m, sq[l]);
        }
    }
    double sumsq = (sq[0] + sq[1]) + (sq[2] + sq[3]);
    for (; k < d; ++k) {
        double m = 0.0;
        for (int64_t i = 0; i < n; ++i) m += (double)streams[i * sd + k];
        m *= inv_n;
        ref[k] = m;
        sumsq = fma(m, m, sumsq);
    }
    const double scale = 1.0 / sqrt(sumsq / (double)d + eps);
    for (k = 0; k < d; ++k) ref[k] = (ref[k] * scale) * (double)norm_w[k];

    for (int64_t r = 0; r < rows; ++r) logit[r] = tanh(dot_lanes(proj_w + r * d, ref, d));
    for (int64_t i = 0; i < n; ++i) {
        const double pre_logit = fma(pre_alpha, logit[i], (double)pre_bias[i]);
        const double post_logit = fma(post_alpha, logit[n + i], (double)post_bias[i]);
        pre[i] = (float)sigmoid_d(pre_logit);
        post[i] = (float)(2.0 * sigmoid_d(post_logit));
    }
    for (int64_t e = 0; e < n * n; ++e) mat[e] = fma(res_alpha, logit[2 * n + e], (double)res_bias[e]);

    /* agg = sum_i pre_i * streams_i: exact products, one rounding. */
    for (k = 0; k < d; ++k) {
        double acc = (double)pre[0] * (double)streams[k];
        for (int64_t i = 1; i < n; ++i) acc = fma((double)pre[i], (double)streams[i * sd + k], acc);
        agg[k] = (float)acc;
    }
    if (agg_norm_w != NULL) agg_norm_inplace(agg, agg_norm_w, agg_norm_eps, d);

    sinkhorn(mat, sums, n, iters);
    for (int64_t e = 0; e < n * n; ++e) res[e] = (float)mat[e];
}

/* Streams are [tokens, n, d] with rows stream_stride floats apart (0 for the
 * broadcast [tokens, d] backbone) and tokens token_stride apart. eps and
 * agg_norm_eps are the Python floats, cast through float32 (montlok.cpp:634,
 * :643); the alphas are the float32 parameters widened to double. */
void orc_mhc_prepare(const float* streams, int64_t stream_stride, int64_t token_stride, const float* norm_w,
                     double eps, const double* proj_w, const float* pre_bias, const float* post_bias,
                     const float* res_bias, float pre_alpha, float post_alpha, float res_alpha, int64_t iters,
                     int64_t tokens, int64_t n, int64_t d, const float* agg_norm_w, double agg_norm_eps, float* agg,
                     float* pre, float* post, float* res) {
    double* scratch = (double*)malloc(sizeof(double) * (size_t)(d + 2 * n + 2 * n * n + n));
    const int it = (int)(iters < (1 << 20) ? iters : (1 << 20));
    for (int64_t t = 0; t < tokens; ++t) {
        mhc_prepare_token(streams + t * token_stride, stream_stride, norm_w, proj_w, pre_bias, post_bias, res_bias,
                          (double)pre_alpha, (double)post_alpha, (double)res_alpha, (double)(float)eps, n, d, it,
                          agg_norm_w, (double)(float)agg_norm_eps, agg + t * d, pre + t * n, post + t * n,
                          res + t * n * n, scratch);
    }
    free(scratch);
}

/* ------------------------------------------------------------------------ */
/* mHC write side: montlok_mhc.h:336-438, ops montlok.cpp:726-758            */
/* ------------------------------------------------------------------------ */

/* new_i = post_i * out + sum_j res_ij * streams_j in double (post term
 * first, then j ascending), one rounding. With `collapsed`, the mean of the
 * rounded new streams in double, one rounding. new_streams may be NULL when
 * only the collapse is wanted. */
void orc_mhc_combine(const float* streams, int64_t stream_stride, int64_t token_stride, const float* res,
                     const float* post, const float* out, int64_t tokens, int64_t n, int64_t d, float* new_streams,
                     float* collapsed) {
    const double inv_n = 1.0 / (double)n;
    float* row = (float*)malloc(sizeof(float) * (size_t)n);
    for (int64_t t = 0; t < tokens; ++t) {
        const float* s = streams + t * token_stride;
        const float* r = res + t * n * n;
        const float* p = post + t * n;
        const float* o = out + t * d;
        for (int64_t k = 0; k < d; ++k) {
            double mean = 0.0;
            for (int64_t i = 0; i < n; ++i) {
                double acc = (double)p[i] * (double)o[k];
                for (int64_t j = 0; j < n; ++j) acc = fma((double)r[i * n + j], (double)s[j * stream_stride + k], acc);
                row[i] = (float)acc;
                mean += (double)row[i];
            }
            if (new_streams != NULL) {
                for (int64_t i = 0; i < n; ++i) new_streams[(t * n + i) * d + k] = row[i];
            }
            if (collapsed != NULL) collapsed[t * d + k] = (float)(mean * inv_n);
        }
    }
    free(row);
}

/* ------------------------------------------------------------------------ */
/* MLA rotary embedding + key assembly: montlok_layers.h:186-234             */
/* ------------------------------------------------------------------------ */

/* rotate_half convention on one vector, fp64, one rounding; out may alias x
 * (montlok_layers.h:190-200). */
static void rope_vector(const float* x, const float* cosine, const float* sine, int64_t rope_dim, float* out) {
    const int64_t half = rope_dim / 2;
    for (int64_t i = 0; i < half; ++i) {
        const double x1 = (double)x[i];
        const double x2 = (double)x[i + half];
        const float o1 = (float)(x1 * (double)cosine[i] - x2 * (double)sine[i]);
        const float o2 = (float)(x2 * (double)cosine[i + half] + x1 * (double)sine[i + half]);
        out[i] = o1;
        out[i + half] = o2;
    }
}

/* q: [B, Lq, H, head_dim] rows q_token_stride apart (rotated in place on the
 * last rope_dim lanes of each head); kv: [B, L, H, nope + head_dim]
 * contiguous; k_rope: [B, L, rope] rows k_rope_token_stride apart;
 * cos/sin: [L, rope]; k: [B, L, H, head_dim] output. Query rows cover the
 * trailing Lq positions (montlok_layers.h:208-227). */
void orc_mla_rope(float* q, int64_t q_token_stride, int64_t q_length, const float* kv, const float* k_rope,
                  int64_t k_rope_token_stride, const float* cosine, const float* sine, float* k, int64_t batch,
                  int64_t length, int64_t heads, int64_t head_dim, int64_t nope_dim) {
    const int64_t rope_dim = head_dim - nope_dim;
    float* rotated = (float*)malloc(sizeof(float) * (size_t)rope_dim);
    const int64_t q_first = length - q_length;
    for (int64_t token = 0; token < batch * length; ++token) {
        const int64_t position = token % length;
        const int64_t sequence = token / length;
        const float* c = cosine + position * rope_dim;
        const float* s = sine + position * rope_dim;
        rope_vector(k_rope + token * k_rope_token_stride, c, s, rope_dim, rotated);
        for (int64_t h = 0; h < heads; ++h) {
            if (position >= q_first) {
                float* qh = q + (sequence * q_length + position - q_first) * q_token_stride + h * head_dim + nope_dim;
                rope_vector(qh, c, s, rope_dim, qh);
            }
            const float* kvh = kv + (token * heads + h) * (nope_dim + head_dim);
            float* kh = k + (token * heads + h) * head_dim;
            memcpy(kh, kvh, sizeof(float) * (size_t)nope_dim);
            memcpy(kh + nope_dim, rotated, sizeof(float) * (size_t)rope_dim);
        }
    }
    free(rotated);
}

/* ------------------------------------------------------------------------ */
/* Linear and attention (the reference calls torch for these)                */
/* ------------------------------------------------------------------------ */

/* out[m, j] = sum_k x[m, k] * w[j, k] (+ bias[j]) in double, one rounding.
 * x rows are x_stride floats apart; out is [M, N] contiguous. */
void orc_linear(const float* x, int64_t x_stride, const float* w, const float* bias, int64_t M, int64_t K, int64_t N,
                float* out) {
    for (int64_t m = 0; m < M; ++m) {
        const float* xr = x + m * x_stride;
        for (int64_t j = 0; j < N; ++j) {
            const float* wr = w + j * K;
            double acc = bias != NULL ? (double)bias[j] : 0.0;
            for (int64_t k = 0; k < K; ++k) acc += (double)xr[k] * (double)wr[k];
            out[m * N + j] = (float)acc;
        }
    }
}

/* Scaled dot-product attention in double, one rounding. q: [B, Lq, H, dh]
 * rows q_ts floats apart per token; k: [B, Lk, H, dh] rows k_ts apart; v
 * likewise with v_ts; out: [B, Lq, H, dh] contiguous. Query i sits at
 * absolute position Lk - Lq + i. mask: 0 none; 1 top-left causal (key j
 * allowed when j <= i, the is_causal convention); 2 bottom-right causal (key
 * j allowed when j <= Lk - Lq + i). Attention semantics of montlok.cpp
 * :1205-1208 and mla.py (reference python/montlok/rdt) :392-413. */
void orc_sdpa(const float* q, int64_t q_ts, const float* k, int64_t k_ts, const float* v, int64_t v_ts, int64_t B,
              int64_t H, int64_t Lq, int64_t Lk, int64_t dh, int mask, double scale, float* out) {
    double* p = (double*)malloc(sizeof(double) * (size_t)Lk);
    for (int64_t b = 0; b < B; ++b) {
        for (int64_t h = 0; h < H; ++h) {
            for (int64_t i = 0; i < Lq; ++i) {
                const float* qi = q + (b * Lq + i) * q_ts + h * dh;
                int64_t last = Lk - 1;
                if (mask == 1) last = i < Lk - 1 ? i : Lk - 1;
                if (mask == 2) last = Lk - Lq + i;
                double mx = -INFINITY;
                for (int64_t j = 0; j <= last; ++j) {
                    const float* kj = k + (b * Lk + j) * k_ts + h * dh;
                    double dot = 0.0;
                    for (int64_t c = 0; c < dh; ++c) dot += (double)qi[c] * (double)kj[c];
                    p[j] = dot * scale;
                    if (p[j] > mx) mx = p[j];
                }
                double denom = 0.0;
                for (int64_t j = 0; j <= last; ++j) {
                    p[j] = exp(p[j] - mx);
                    denom += p[j];
                }
                float* oi = out + ((b * Lq + i) * H + h) * dh;
                for (int64_t c = 0; c < dh; ++c) {
                    double acc = 0.0;
                    for (int64_t j = 0; j <= last; ++j) acc += p[j] * (double)v[(b * Lk + j) * v_ts + h * dh + c];
                    oi[c] = (float)(acc / denom);
                }
            }
        }
    }
    free(p);
}
