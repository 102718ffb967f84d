// Thin C entry points over the reference's header-only CPU kernels
// (rdt4quant_cpu/montlok_{types,kernel,mhc,layers}.h), compiled from the
// files where they lie in the reference checkout by oracle/Makefile into
// oracle/_ref/. Nothing here re-implements a kernel: every function fills the
// reference's own plan struct and calls the reference's own kernel over all of
// its work items, the way the reference's PyTorch glue does
// (rdt4quant_cpu/montlok.cpp). The library is test infrastructure: it writes
// the golden vectors and serves as the timed CPU baseline; it never runs on
// the product path.
//
// Work items are spread over OpenMP threads with dynamic scheduling, the
// same decomposition as montlok.cpp:200-227 (parallel_items): recurrence work
// items, 4-token mHC blocks, and one row / token per item elsewhere.

#include <omp.h>

#include <cstdint>
#include <vector>

#include "montlok_layers.h"

using namespace montlok;

extern "C" {

int ref_vec_bytes() { return MONTLOK_VEC_BYTES; }

int ref_max_threads() { return omp_get_max_threads(); }

void ref_set_threads(int threads) { omp_set_num_threads(threads > 0 ? threads : 1); }

// montlok.cpp:915-938 (rms_norm): eps is cast through float there.
void ref_rms_norm(const float* x, int64_t row_stride, const float* w, double eps, int64_t dim, int64_t groups,
                  int64_t rows, float* out) {
    const double eps_f = static_cast<double>(static_cast<float>(eps));
#pragma omp parallel for schedule(dynamic, 64)
    for (int64_t row = 0; row < rows; ++row) {
        rms_norm_rows(x, row_stride, w, eps_f, dim, groups, row, row + 1, out);
    }
}

// montlok.cpp:978-1007 (add_rms_norm).
void ref_add_rms_norm(const float* left, const float* right, const float* w, double eps, int64_t dim,
                      int64_t groups, int64_t rows, float* residual, float* normalized) {
    const double eps_f = static_cast<double>(static_cast<float>(eps));
#pragma omp parallel for schedule(dynamic, 64)
    for (int64_t row = 0; row < rows; ++row) {
        add_rms_norm_rows(left, right, w, eps_f, dim, groups, row, row + 1, residual, normalized);
    }
}

// montlok.cpp:1057-1082 (layer_norm); bias may be null.
void ref_layer_norm(const float* x, int64_t row_stride, const float* w, const float* bias, double eps, int64_t dim,
                    int64_t rows, float* out) {
    const double eps_f = static_cast<double>(static_cast<float>(eps));
#pragma omp parallel for schedule(dynamic, 64)
    for (int64_t row = 0; row < rows; ++row) {
        layer_norm_rows(x, row_stride, w, bias, eps_f, dim, row, row + 1, out);
    }
}

// montlok.cpp:942-963 (swiglu).
void ref_swiglu(const float* x, int64_t row_stride, int64_t hidden, int64_t rows, float* out) {
#pragma omp parallel for schedule(dynamic, 64)
    for (int64_t row = 0; row < rows; ++row) {
        swiglu_rows(x, row_stride, hidden, row, row + 1, out);
    }
}

// montlok.cpp:279-299: per-token (alpha, beta, gamma) from (adt, dt, trap_logit).
void ref_step_coefficients(const float* adt, const float* dt, const float* trap, int64_t count, float* alpha,
                           float* beta, float* gamma) {
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < count; ++i) {
        const StepCoefficients c = step_coefficients(adt[i], dt[i], trap[i]);
        alpha[i] = c.alpha;
        beta[i] = c.beta;
        gamma[i] = c.gamma;
    }
}

// montlok_kernel.h:433-457 over every work item (montlok.cpp:229-237).
// Strides are element strides of the leading [B, L, H] dimensions.
void ref_siso(int64_t B, int64_t L, int64_t H, int64_t N, int64_t D, const float* q, const int64_t* qs,
              const float* k, const int64_t* ks, const float* v, const int64_t* vs, const float* gate,
              const int64_t* gs, int gate_logits, const float* alpha, const float* beta, const float* gamma,
              const float* skip, float* out, const int64_t* os) {
    SisoPlan p{};
    p.B = B;
    p.L = L;
    p.H = H;
    p.N = N;
    p.D = D;
    p.q = q;
    p.qs = {qs[0], qs[1], qs[2]};
    p.k = k;
    p.ks = {ks[0], ks[1], ks[2]};
    p.v = v;
    p.vs = {vs[0], vs[1], vs[2]};
    p.gate = gate;
    p.gs = {gs[0], gs[1], gs[2]};
    p.gate_logits = gate_logits != 0;
    p.alpha = alpha;
    p.beta = beta;
    p.gamma = gamma;
    p.skip = skip;
    p.out = out;
    p.os = {os[0], os[1], os[2]};
    const int64_t items = siso_work_items(p);
#pragma omp parallel
    {
        std::vector<float> scratch(static_cast<size_t>(siso_scratch_floats(p)));
#pragma omp for schedule(dynamic, 1)
        for (int64_t item = 0; item < items; ++item) {
            siso_run_work_item(p, item, scratch.data());
        }
    }
}

// Phases A, B, C of the fused pre-processing (montlok.cpp:443-461).
// q, k: [B, L, H, N]; alpha/beta/gamma: [B, L, H]; angle_term [B, L, H, max(R,1)]
// and cum [B, H, max(R,1), L] are workspaces.
void ref_prep(int64_t B, int64_t L, int64_t W, const float* proj, int64_t proj_sb, int64_t proj_st,
              int64_t d_inner, int64_t N, int64_t G, int64_t H, int64_t D, int64_t R, const float* b_bias,
              const float* c_bias, const float* b_norm_w, const float* c_norm_w, double b_eps, double c_eps,
              const float* dt_bias, double a_floor, float* q, float* k, float* alpha, float* beta, float* gamma,
              float* angle_term, float* cum) {
    PrepPlan p{};
    p.B = B;
    p.L = L;
    p.W = W;
    p.proj = proj;
    p.proj_sb = proj_sb;
    p.proj_st = proj_st;
    p.d_inner = d_inner;
    p.N = N;
    p.G = G;
    p.H = H;
    p.D = D;
    p.R = R;
    p.b_bias = b_bias;
    p.c_bias = c_bias;
    p.b_norm_w = b_norm_w;
    p.c_norm_w = c_norm_w;
    p.b_eps = static_cast<float>(b_eps);
    p.c_eps = static_cast<float>(c_eps);
    p.dt_bias = dt_bias;
    p.a_floor = static_cast<float>(a_floor);
    p.q = q;
    p.k = k;
    p.alpha = alpha;
    p.beta = beta;
    p.gamma = gamma;
    p.angle_term = angle_term;
    p.cum = cum;
    const int64_t tokens = B * L;
#pragma omp parallel
    {
        std::vector<float> scratch(static_cast<size_t>(prep_scratch_floats(p)));
#pragma omp for schedule(dynamic, 16)
        for (int64_t token = 0; token < tokens; ++token) {
            prep_token(p, token / L, token % L, scratch.data());
        }
    }
    if (R > 0) {
#pragma omp parallel for schedule(dynamic, 16)
        for (int64_t chain = 0; chain < B * H * R; ++chain) {
            prep_chain(p, chain);
        }
#pragma omp parallel for schedule(dynamic, 16)
        for (int64_t token = 0; token < tokens; ++token) {
            prep_rotate(p, token / L, token % L);
        }
    }
}

// mamba3_siso_forward (montlok.cpp:333-492) with an empty gate: the silu of
// the z lanes is evaluated inside the recurrence. Returns [B, L, d_inner].
// Workspaces: q, k [B*L*H*N]; coef [3*B*L*H]; angle_term, cum [B*L*H*max(R,1)].
void ref_mamba3_siso_forward(int64_t B, int64_t L, const float* proj, int64_t proj_sb, int64_t proj_st,
                             int64_t N, int64_t G, int64_t H, int64_t D, int64_t R, const float* b_bias,
                             const float* c_bias, const float* b_norm_w, const float* c_norm_w, double b_eps,
                             double c_eps, const float* dt_bias, const float* skip, double a_floor, float* q,
                             float* k, float* coef, float* angle_term, float* cum, float* out) {
    const int64_t d_inner = H * D;
    const int64_t W = 2 * d_inner + 2 * G * N + 3 * H + R;
    const int64_t BLH = B * L * H;
    ref_prep(B, L, W, proj, proj_sb, proj_st, d_inner, N, G, H, D, R, b_bias, c_bias, b_norm_w, c_norm_w, b_eps,
             c_eps, dt_bias, a_floor, q, k, coef, coef + BLH, coef + 2 * BLH, angle_term, cum);
    const int64_t qs[3] = {L * H * N, H * N, N};
    const int64_t vs[3] = {proj_sb, proj_st, D};
    const int64_t os[3] = {L * d_inner, d_inner, D};
    ref_siso(B, L, H, N, D, q, qs, k, qs, proj + d_inner, vs, proj, vs, 1, coef, coef + BLH, coef + 2 * BLH, skip,
             out, os);
}

static MhcPlan make_mhc_plan(const float* streams, int64_t stream_stride, int64_t token_stride, const float* norm_w,
                             const double* proj_w, const float* pre_bias, const float* post_bias,
                             const float* res_bias, double pre_alpha, double post_alpha, double res_alpha,
                             double eps, int64_t tokens, int64_t n, int64_t d, int64_t iters,
                             const float* agg_norm_w, double agg_norm_eps, float* agg, float* pre, float* post,
                             float* res) {
    MhcPlan p{};
    p.streams = streams;
    p.stream_stride = stream_stride;
    p.token_stride = token_stride;
    p.norm_w = norm_w;
    p.proj_w = proj_w;
    p.pre_bias = pre_bias;
    p.post_bias = post_bias;
    p.res_bias = res_bias;
    p.pre_alpha = pre_alpha;
    p.post_alpha = post_alpha;
    p.res_alpha = res_alpha;
    // montlok.cpp:634 and :643: the Python float eps meets a float32 tensor.
    p.eps = static_cast<double>(static_cast<float>(eps));
    p.tokens = tokens;
    p.n = n;
    p.d = d;
    p.sinkhorn_iters = static_cast<int>(iters < (1 << 20) ? iters : (1 << 20));
    p.agg = agg;
    p.agg_norm_w = agg_norm_w;
    p.agg_norm_eps = static_cast<double>(static_cast<float>(agg_norm_eps));
    p.pre = pre;
    p.post = post;
    p.res = res;
    return p;
}

// mhc_prepare (montlok.cpp:659-691). The alphas are the float32 parameter
// values widened to double (montlok.cpp:601-605).
void ref_mhc_prepare(const float* streams, int64_t stream_stride, int64_t token_stride, const float* norm_w,
                     double eps, const double* proj_w, const float* pre_bias, const float* post_bias,
                     const float* res_bias, float pre_alpha, float post_alpha, float res_alpha, int64_t iters,
                     int64_t tokens, int64_t n, int64_t d, const float* agg_norm_w, double agg_norm_eps, float* agg,
                     float* pre, float* post, float* res) {
    const MhcPlan p = make_mhc_plan(streams, stream_stride, token_stride, norm_w, proj_w, pre_bias, post_bias,
                                    res_bias, pre_alpha, post_alpha, res_alpha, eps, tokens, n, d, iters, agg_norm_w,
                                    agg_norm_eps, agg, pre, post, res);
    const int64_t blocks = (tokens + kMhcTokenBlock - 1) / kMhcTokenBlock;
#pragma omp parallel
    {
        std::vector<double> scratch(static_cast<size_t>(mhc_scratch_doubles(p)));
#pragma omp for schedule(dynamic, 4)
        for (int64_t block = 0; block < blocks; ++block) {
            const int64_t begin = block * kMhcTokenBlock;
            const int64_t end = begin + kMhcTokenBlock < tokens ? begin + kMhcTokenBlock : tokens;
            mhc_prepare_range(p, begin, end, scratch.data());
        }
    }
}

// mhc_combine / mhc_combine_collapse (montlok.cpp:726-758). With collapse
// set, new_streams is ignored and only the mean over streams is written.
void ref_mhc_combine(const float* streams, int64_t stream_stride, int64_t token_stride, const float* res,
                     const float* post, const float* out, int64_t tokens, int64_t n, int64_t d, float* new_streams,
                     float* collapsed, int collapse_only) {
    MhcCombinePlan c{};
    c.streams = streams;
    c.stream_stride = stream_stride;
    c.token_stride = token_stride;
    c.res = res;
    c.post = post;
    c.out = out;
    c.new_streams = new_streams;
    c.collapsed = collapsed;
    c.n = n;
    c.d = d;
    if (collapse_only) {
#pragma omp parallel
        {
            std::vector<float> scratch(static_cast<size_t>(n * d));
#pragma omp for schedule(dynamic, 64)
            for (int64_t token = 0; token < tokens; ++token) {
                mhc_combine_collapse_range(c, token, token + 1, scratch.data());
            }
        }
    } else {
#pragma omp parallel for schedule(dynamic, 64)
        for (int64_t token = 0; token < tokens; ++token) {
            mhc_combine_range(c, token, token + 1);
        }
    }
}

// mhc_combine_prepare (montlok.cpp:763-802): write of this residual fused
// with the read of the next one, whose parameters follow.
void ref_mhc_combine_prepare(const float* streams, int64_t stream_stride, int64_t token_stride, const float* res,
                             const float* post, const float* out, const float* norm_w, double eps,
                             const double* proj_w, const float* pre_bias, const float* post_bias,
                             const float* res_bias, float pre_alpha, float post_alpha, float res_alpha,
                             int64_t iters, int64_t tokens, int64_t n, int64_t d, const float* agg_norm_w,
                             double agg_norm_eps, float* new_streams, float* agg, float* pre_out, float* post_out,
                             float* res_out) {
    MhcCombinePlan c{};
    c.streams = streams;
    c.stream_stride = stream_stride;
    c.token_stride = token_stride;
    c.res = res;
    c.post = post;
    c.out = out;
    c.new_streams = new_streams;
    c.collapsed = nullptr;
    c.n = n;
    c.d = d;
    MhcPlan p = make_mhc_plan(new_streams, d, n * d, norm_w, proj_w, pre_bias, post_bias, res_bias, pre_alpha,
                              post_alpha, res_alpha, eps, tokens, n, d, iters, agg_norm_w, agg_norm_eps, agg,
                              pre_out, post_out, res_out);
    const int64_t blocks = (tokens + kMhcTokenBlock - 1) / kMhcTokenBlock;
#pragma omp parallel
    {
        std::vector<double> scratch(static_cast<size_t>(mhc_scratch_doubles(p)));
#pragma omp for schedule(dynamic, 4)
        for (int64_t block = 0; block < blocks; ++block) {
            const int64_t begin = block * kMhcTokenBlock;
            const int64_t end = begin + kMhcTokenBlock < tokens ? begin + kMhcTokenBlock : tokens;
            mhc_combine_prepare_range(c, p, begin, end, scratch.data());
        }
    }
}

// mla_rope_qk (montlok.cpp:1093-1154): rotates q in place and writes k.
void ref_mla_rope(float* q, int64_t q_token_stride, int64_t q_head_stride, int64_t q_length, const float* kv,
                  int64_t kv_token_stride, int64_t kv_head_stride, const float* k_rope, int64_t k_rope_token_stride,
                  const float* cosine, const float* sine, float* k, int64_t batch, int64_t length, int64_t heads,
                  int64_t head_dim, int64_t nope_dim) {
    MlaRopePlan p{};
    p.q = q;
    p.q_token_stride = q_token_stride;
    p.q_head_stride = q_head_stride;
    p.q_length = q_length;
    p.kv = kv;
    p.kv_token_stride = kv_token_stride;
    p.kv_head_stride = kv_head_stride;
    p.k_rope = k_rope;
    p.k_rope_token_stride = k_rope_token_stride;
    p.cosine = cosine;
    p.sine = sine;
    p.k = k;
    p.length = length;
    p.heads = heads;
    p.head_dim = head_dim;
    p.nope_dim = nope_dim;
    p.rope_dim = head_dim - nope_dim;
#pragma omp parallel
    {
        std::vector<float> scratch(static_cast<size_t>(p.rope_dim));
#pragma omp for schedule(dynamic, 64)
        for (int64_t token = 0; token < batch * length; ++token) {
            mla_rope_range(p, token, token + 1, scratch.data());
        }
    }
}

}  // extern "C"
