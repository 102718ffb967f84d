"""Pins of the CPU oracle (oracle/mlk_oracle.c), CPU only.

Three kinds of pin, chosen so that a plausible slip in the oracle (a dropped
term, a wrong index, an operand swap, a different rounding) fails at least one:

1. Golden vectors written by the reference's own compiled kernels
   (tests/golden/make_golden.py): the oracle must reproduce them bit for bit.
2. Live cross-checks against the compiled reference (oracle/_ref) on fresh
   random cases, where that library is built (the build container).
3. Mathematics the reference does not state in code: fp64 closed forms,
   brute-force recurrences, an independent quadratic (segment-sum) form of the
   Mamba-3 scan, Sinkhorn invariants, rotation invariants, and torch's float64
   CPU routines for GEMM and attention.
"""

from __future__ import annotations

import math

import numpy as np
import pytest

from helpers import assert_bitwise, assert_close, rel_err
from oracle import Reference, reference_available


# --------------------------------------------------------------- golden vectors


def test_golden_norms(oracle, golden):
    g = golden("norms")
    for i in range(4):
        groups, eps = g[f"rms{i}_meta"]
        x, w = g[f"rms{i}_x"], g[f"rms{i}_w"]
        assert_bitwise(oracle.rms_norm(x, w, eps, int(groups)), g[f"rms{i}_out"], f"rms{i}")
        res, nrm = oracle.add_rms_norm(x, g[f"rms{i}_right"], w, eps, int(groups))
        assert_bitwise(res, g[f"rms{i}_residual"], f"add_rms{i} residual")
        assert_bitwise(nrm, g[f"rms{i}_normalized"], f"add_rms{i} normalized")
    for i in range(3):
        b = g.get(f"ln{i}_b")
        assert_bitwise(oracle.layer_norm(g[f"ln{i}_x"], g[f"ln{i}_w"], b, 1e-5), g[f"ln{i}_out"], f"ln{i}")
    for i in range(2):
        assert_bitwise(oracle.swiglu(g[f"swiglu{i}_x"]), g[f"swiglu{i}_out"], f"swiglu{i}")


def test_golden_siso(oracle, golden):
    g = golden("siso")
    for i in range(4):
        c = {k[len(f"c{i}_"):]: v for k, v in g.items() if k.startswith(f"c{i}_")}
        al, be, ga = oracle.step_coefficients(c["adt"], c["dt"], c["trap"])
        assert_bitwise(al, c["alpha"], "alpha")
        assert_bitwise(be, c["beta"], "beta")
        assert_bitwise(ga, c["gamma"], "gamma")
        out = oracle.siso(c["q"], c["k"], c["v"], c["gate"], al, be, ga, c["skip"], gate_logits=False)
        assert_bitwise(out, c["out"], f"siso{i}")
        out = oracle.siso(c["q"], c["k"], c["v"], c["z"], al, be, ga, c["skip"], gate_logits=True)
        assert_bitwise(out, c["out_silu"], f"siso{i} in-kernel silu")


def _mamba_case(g, i):
    c = {k[len(f"c{i}_"):]: v for k, v in g.items() if k.startswith(f"c{i}_")}
    N, G, H, D, R = (int(v) for v in c["geom"])
    return c, (N, G, H, D, R)


def test_golden_mamba_prep_and_forward(oracle, golden):
    g = golden("mamba_forward")
    for i in range(5):
        c, geom = _mamba_case(g, i)
        args = (c["b_bias"], c["c_bias"], c["b_norm_w"], c["c_norm_w"], 1e-5, 1e-5, c["dt_bias"])
        q, k, al, be, ga = oracle.prep(c["proj"], *geom, *args, 1e-4)
        for name, a, e in (("q", q, c["q"]), ("k", k, c["k"]), ("alpha", al, c["alpha"]), ("beta", be, c["beta"]),
                           ("gamma", ga, c["gamma"])):
            assert_bitwise(a, e, f"prep{i} {name}")
        out = oracle.mamba3_siso_forward(c["proj"], *geom, *args, c["skip"], 1e-4)
        assert_bitwise(out, c["out"], f"mamba3_siso_forward{i}")


def test_golden_mhc(oracle, golden):
    g = golden("mhc")
    a_pre, a_post, a_res = (float(v) for v in g["alphas"])
    for i in range(6):
        c = {k[len(f"c{i}_"):]: v for k, v in g.items() if k.startswith(f"c{i}_")}
        n, d, iters = (int(v) for v in c["meta"])
        params = (c["norm_w"], 1e-5, c["proj_w"], c["pre_bias"], c["post_bias"], c["res_bias"], a_pre, a_post, a_res,
                  iters)
        agg, pre, post, res = oracle.mhc_prepare(c["streams"], *params)
        for name, a, e in (("agg", agg, c["agg"]), ("pre", pre, c["pre"]), ("post", post, c["post"]),
                           ("res", res, c["res"])):
            assert_bitwise(a, e, f"mhc{i} {name}")
        assert_bitwise(oracle.mhc_prepare(c["streams"], *params, 0, c["agg_norm_w"], 1e-6)[0], c["agg_normed"],
                       f"mhc{i} agg_norm")
        b = oracle.mhc_prepare(np.ascontiguousarray(c["streams"][:, :, 0, :]), *params, n)
        for name, a in zip(("agg", "pre", "post", "res"), b):
            assert_bitwise(a, c[f"bcast_{name}"], f"mhc{i} broadcast {name}")
        assert_bitwise(oracle.mhc_combine(c["streams"], c["res"], c["post"], c["out"]), c["new"], f"combine{i}")
        col = oracle.mhc_combine(c["streams"], c["res"], c["post"], c["out"], collapse=True, materialize=False)
        assert_bitwise(col, c["collapsed"], f"collapse{i}")
        # combine_prepare = combine, then prepare of the new streams.
        nxt = oracle.mhc_prepare(c["new"], *params)
        for name, a in zip(("agg", "pre", "post", "res"), nxt):
            assert_bitwise(a, c[f"next_{name}"], f"combine_prepare{i} {name}")
        assert_bitwise(c["new"], c["next_new"], f"combine_prepare{i} streams")


def test_golden_rope(oracle, golden):
    g = golden("rope")
    for i in range(5):
        c = {k[len(f"c{i}_"):]: v for k, v in g.items() if k.startswith(f"c{i}_")}
        q, k = oracle.mla_rope(c["q"], c["kv"], c["k_rope"], c["cos"], c["sin"], int(c["nope"][0]))
        assert_bitwise(q, c["q_out"], f"rope{i} q")
        assert_bitwise(k, c["k_out"], f"rope{i} k")


# ------------------------------------------------------- live compiled reference


needs_ref = pytest.mark.skipif(not reference_available("avx2"),
                               reason="oracle/_ref is built only where the reference exists")


@needs_ref
@pytest.mark.parametrize("seed", [1, 2])
def test_live_reference_mamba(oracle, seed):
    ref = Reference("avx2")
    rng = np.random.default_rng(seed)
    for N, G, H, D, R in [(16, 1, 4, 32, 4), (64, 1, 4, 64, 16), (12, 2, 4, 16, 5)]:
        B, L = 2, 33
        W = 2 * H * D + 2 * G * N + 3 * H + R
        proj = rng.standard_normal((B, L, W)).astype(np.float32)
        bb = (1 + 0.3 * rng.standard_normal((H, N))).astype(np.float32)
        cb = (1 + 0.3 * rng.standard_normal((H, N))).astype(np.float32)
        bw = (rng.random(N) + 0.5).astype(np.float32)
        cw = (rng.random(N) + 0.5).astype(np.float32)
        dtb = (rng.standard_normal(H) - 2).astype(np.float32)
        skip = rng.standard_normal(H).astype(np.float32)
        args = (N, G, H, D, R, bb, cb, bw, cw, 1e-5, 1e-5, dtb, skip, 1e-4)
        assert_bitwise(oracle.mamba3_siso_forward(proj, *args), ref.mamba3_siso_forward(proj, *args), "forward")


@needs_ref
def test_live_reference_mhc(oracle):
    ref = Reference("avx2")
    rng = np.random.default_rng(5)
    for n, d in [(4, 128), (4, 256), (2, 40)]:
        s = (rng.standard_normal((2, 21, n, d)) * 1.5).astype(np.float32)
        nw = (rng.random(d) + 0.5).astype(np.float32)
        pw = (rng.standard_normal((2 * n + n * n, d)) * 4 / np.sqrt(d)).astype(np.float32).astype(np.float64)
        pb, qb = rng.standard_normal(n).astype(np.float32), rng.standard_normal(n).astype(np.float32)
        rb = rng.standard_normal((n, n)).astype(np.float32)
        params = (nw, 1e-5, pw, pb, qb, rb, 0.7, 0.7, 0.7, 20)
        for a, e in zip(oracle.mhc_prepare(s, *params), ref.mhc_prepare(s, *params)):
            assert_bitwise(a, e, f"mhc n{n} d{d}")


# ---------------------------------------------------------- mathematical pins


def test_rms_norm_closed_form_and_scale_invariance(oracle):
    rng = np.random.default_rng(0)
    x = rng.standard_normal((50, 64)).astype(np.float32) * 3
    w = (rng.random(64) + 0.5).astype(np.float32)
    for groups in (1, 4, 8):
        xg = x.astype(np.float64).reshape(50, groups, -1)
        eps = float(np.float32(1e-5))
        expect = (xg / np.sqrt((xg ** 2).mean(-1, keepdims=True) + eps)).reshape(50, 64) * w
        assert rel_err(oracle.rms_norm(x, w, 1e-5, groups), expect) < 1e-7
    # A group scaled by a power of two normalises to the same values (eps ~ 0).
    out1 = oracle.rms_norm(x, w, 1e-30, 4)
    x2 = x.copy()
    x2[:, 16:32] *= 8.0
    assert_bitwise(oracle.rms_norm(x2, w, 1e-30, 4), out1, "rms scale invariance")


def test_layer_norm_closed_form(oracle):
    rng = np.random.default_rng(1)
    x = (rng.standard_normal((40, 96)) * 2 + 0.5).astype(np.float32)
    w = (rng.random(96) + 0.5).astype(np.float32)
    b = rng.standard_normal(96).astype(np.float32)
    xd = x.astype(np.float64)
    mean = xd.mean(-1, keepdims=True)
    var = ((xd - mean) ** 2).mean(-1, keepdims=True)
    expect = (xd - mean) / np.sqrt(var + float(np.float32(1e-5))) * w + b
    assert rel_err(oracle.layer_norm(x, w, b, 1e-5), expect) < 1e-7


def _siso_bruteforce(q, k, v, gate, al, be, ga, skip):
    """fp64 recurrence S_t = a S_{t-1} + b k_{t-1} v_{t-1}^T + g k_t v_t^T, zero start."""
    B, L, H, N = q.shape
    D = v.shape[-1]
    out = np.zeros((B, L, H, D))
    for b in range(B):
        for h in range(H):
            S = np.zeros((N, D))
            for t in range(L):
                S = al[b, t, h] * S + ga[b, t, h] * np.outer(k[b, t, h], v[b, t, h])
                if t > 0:
                    S += be[b, t, h] * np.outer(k[b, t - 1, h], v[b, t - 1, h])
                out[b, t, h] = (q[b, t, h] @ S + skip[h] * v[b, t, h]) * gate[b, t, h]
    return out


def _coefficients(rng, shape):
    dt = np.log1p(np.exp(rng.standard_normal(shape) - 2.0)).astype(np.float32)
    adt = (-(np.abs(rng.standard_normal(shape)) + 0.5) * dt).astype(np.float32)
    trap = rng.standard_normal(shape).astype(np.float32)
    return adt, dt, trap


def test_siso_against_fp64_bruteforce_and_closed_forms(oracle):
    rng = np.random.default_rng(2)
    B, L, H, N, D = 2, 17, 3, 8, 16
    q = (rng.standard_normal((B, L, H, N)) * 0.5).astype(np.float32)
    k = (rng.standard_normal((B, L, H, N)) * 0.5).astype(np.float32)
    v = rng.standard_normal((B, L, H, D)).astype(np.float32)
    gate = rng.standard_normal((B, L, H, D)).astype(np.float32)
    skip = rng.standard_normal(H).astype(np.float32)
    al, be, ga = oracle.step_coefficients(*_coefficients(rng, (B, L, H)))
    expect = _siso_bruteforce(q, k, v, gate, al, be, ga, skip)
    out = oracle.siso(q, k, v, gate, al, be, ga, skip)
    assert np.abs(out - expect).max() <= 2e-6 * (1 + np.abs(expect).max())
    # L = 1: y = (gamma (q . k) v + D v) * gate.
    y1 = oracle.siso(q[:, :1], k[:, :1], v[:, :1], gate[:, :1], al[:, :1], be[:, :1], ga[:, :1], skip)
    closed = ((ga[:, :1, :, None] * (q[:, :1] * k[:, :1]).sum(-1, keepdims=True).astype(np.float64)) * v[:, :1]
              + skip[None, None, :, None] * v[:, :1]) * gate[:, :1]
    assert rel_err(y1, closed) < 1e-6
    # dt -> 0: no state input, y = D v * gate.
    zeros = np.zeros_like(ga)
    y0 = oracle.siso(q, k, v, gate, np.ones_like(al), zeros, zeros, skip)
    assert rel_err(y0, skip[None, None, :, None] * v * gate) < 1e-6


def test_coefficient_special_cases(oracle):
    # trap -> +inf: beta = 0, gamma = dt; trap -> -inf: gamma = 0, beta = dt * alpha.
    dt = np.array([0.01, 0.05, 0.1], np.float32)
    adt = np.array([-0.02, -0.1, -0.3], np.float32)
    al, be, ga = oracle.step_coefficients(adt, dt, np.full(3, 100.0, np.float32))
    assert np.all(be == 0) and np.array_equal(ga, dt) and np.allclose(al, np.exp(adt), rtol=1e-7)
    al, be, ga = oracle.step_coefficients(adt, dt, np.full(3, -100.0, np.float32))
    assert np.all(ga == 0) and np.allclose(be, dt * al, rtol=1e-7)


def _quadratic_mamba(proj, N, G, H, D, R, bb, cb, bw, cw, dtb, skip, a_floor, eps=1e-5):
    """The quadratic (segment-sum) form of the Mamba-3 SISO layer in fp64: an
    algorithm independent of the recurrence (python/montlok/rdt/mamba3.py
    :199-266, restated in numpy)."""
    B, L, W = proj.shape
    p = proj.astype(np.float64)
    di = H * D
    z = p[..., :di].reshape(B, L, H, D)
    x = p[..., di:2 * di].reshape(B, L, H, D)
    o = 2 * di
    braw = p[..., o:o + G * N].reshape(B, L, G, N)
    craw = p[..., o + G * N:o + 2 * G * N].reshape(B, L, G, N)
    o += 2 * G * N
    raw_dt, raw_a, raw_trap = p[..., o:o + H], p[..., o + H:o + 2 * H], p[..., o + 2 * H:o + 3 * H]
    raw_ang = p[..., o + 3 * H:o + 3 * H + R]

    def bcnorm(v, w):
        return v / np.sqrt((v ** 2).mean(-1, keepdims=True) + eps) * w

    rep = H // G
    bn = np.repeat(bcnorm(braw, bw), rep, axis=2)
    cn = np.repeat(bcnorm(craw, cw), rep, axis=2)
    k0 = bn + bb.reshape(1, 1, H, N)
    q0 = cn + cb.reshape(1, 1, H, N)
    dt = np.logaddexp(0.0, raw_dt + dtb)
    a = -np.maximum(np.maximum(raw_a, 0) + 1.0 / (1.0 - np.minimum(raw_a, 0)), a_floor)
    adt = a * dt
    trap = 1.0 / (1.0 + np.exp(-raw_trap))
    ang = np.tanh(raw_ang)[:, :, None, :] * math.pi * dt[..., None]
    cum = np.cumsum(ang, axis=1)

    def rotate(v):
        out = v.copy()
        for r in range(R):
            c, s = np.cos(cum[..., r]), np.sin(cum[..., r])
            l, rr = v[..., 2 * r], v[..., 2 * r + 1]
            out[..., 2 * r] = l * c - rr * s
            out[..., 2 * r + 1] = l * s + rr * c
        return out

    q, k = rotate(q0), rotate(k0)
    sdt = np.concatenate([dt[:, 1:], np.zeros_like(dt[:, :1])], 1)
    strap = np.concatenate([trap[:, 1:], np.zeros_like(trap[:, :1])], 1)
    sgamma = sdt * (1 - strap)
    scale = dt * trap + sgamma
    qk_skip = (q0 * k0).sum(-1) * sgamma
    cs = np.cumsum(adt, axis=1)  # [B, L, H]
    decay = np.exp(cs[:, :, None, :] - cs[:, None, :, :])  # [B, t, s, H]
    mask = np.tril(np.ones((L, L)))[None, :, :, None]
    qk = np.einsum("bthn,bshn->btsh", q, k * scale[..., None]) * decay * mask
    y = np.einsum("btsh,bshd->bthd", qk, x) + skip.reshape(1, 1, H, 1) * x - x * qk_skip[..., None]
    return (y * z / (1 + np.exp(-z))).reshape(B, L, di)


def test_mamba_forward_against_quadratic_form(oracle):
    rng = np.random.default_rng(3)
    for N, G, H, D, R in [(16, 1, 4, 16, 4), (8, 2, 4, 8, 2), (6, 1, 3, 12, 0)]:
        B, L = 2, 21
        W = 2 * H * D + 2 * G * N + 3 * H + R
        proj = rng.standard_normal((B, L, W)).astype(np.float32)
        bb = (1 + 0.3 * rng.standard_normal((H, N))).astype(np.float32)
        cb = (1 + 0.3 * rng.standard_normal((H, N))).astype(np.float32)
        bw = (rng.random(N) + 0.5).astype(np.float32)
        cw = (rng.random(N) + 0.5).astype(np.float32)
        dtb = (rng.standard_normal(H) - 2).astype(np.float32)
        skip = rng.standard_normal(H).astype(np.float32)
        out = oracle.mamba3_siso_forward(proj, N, G, H, D, R, bb, cb, bw, cw, 1e-5, 1e-5, dtb, skip, 1e-4)
        expect = _quadratic_mamba(proj, N, G, H, D, R, bb, cb, bw, cw, dtb, skip, 1e-4)
        assert np.abs(out - expect).max() <= 2e-5 * (1 + np.abs(expect).max()), (N, G, H, D, R)


def test_mamba_step_sequence_identity(oracle):
    """Stepping T tokens from a zero state equals the sequence op over T tokens."""
    rng = np.random.default_rng(4)
    for N, G, H, D, R in [(16, 1, 4, 16, 4), (64, 1, 2, 64, 16), (6, 1, 3, 12, 1)]:
        S, T = 3, 9
        W = 2 * H * D + 2 * G * N + 3 * H + R
        proj = rng.standard_normal((S, T, W)).astype(np.float32)
        bb = (1 + 0.3 * rng.standard_normal((H, N))).astype(np.float32)
        cb = (1 + 0.3 * rng.standard_normal((H, N))).astype(np.float32)
        bw = (rng.random(N) + 0.5).astype(np.float32)
        cw = (rng.random(N) + 0.5).astype(np.float32)
        dtb = (rng.standard_normal(H) - 2).astype(np.float32)
        skip = rng.standard_normal(H).astype(np.float32)
        args = (N, G, H, D, R, bb, cb, bw, cw, 1e-5, 1e-5, dtb, skip, 1e-4)
        seq = oracle.mamba3_siso_forward(proj, *args)
        state = dict(ssm=np.zeros((S, H, N, D), np.float32), k_prev=np.zeros((S, H, N), np.float32),
                     v_prev=np.zeros((S, H, D), np.float32), angle=np.zeros((S, H, max(R, 1))), started=0)
        for t in range(T):
            y = oracle.mamba3_step(np.ascontiguousarray(proj[:, t]), state, *args)
            assert_bitwise(y, seq[:, t], f"step {t}")


def test_mamba_step_threads_equal_one_call(oracle):
    """The streams split over OpenMP threads (the CPU baseline's form) give the one-call result and states."""
    rng = np.random.default_rng(5)
    N, G, H, D, R = 16, 1, 4, 16, 4
    S = 37
    W = 2 * H * D + 2 * G * N + 3 * H + R
    bb, cb = (1 + 0.3 * rng.standard_normal((2, H, N))).astype(np.float32)
    bw, cw = (rng.random((2, N)) + 0.5).astype(np.float32)
    dtb = (rng.standard_normal(H) - 2).astype(np.float32)
    skip = rng.standard_normal(H).astype(np.float32)
    args = (N, G, H, D, R, bb, cb, bw, cw, 1e-5, 1e-5, dtb, skip, 1e-4)
    start = dict(ssm=rng.standard_normal((S, H, N, D)).astype(np.float32) * 0.1,
                 k_prev=rng.standard_normal((S, H, N)).astype(np.float32),
                 v_prev=rng.standard_normal((S, H, D)).astype(np.float32),
                 angle=rng.random((S, H, R)) * 6.0, started=1)
    one = {k: (v.copy() if isinstance(v, np.ndarray) else v) for k, v in start.items()}
    many = {k: (v.copy() if isinstance(v, np.ndarray) else v) for k, v in start.items()}
    for t in range(3):
        proj = rng.standard_normal((S, W)).astype(np.float32)
        y1 = oracle.mamba3_step(proj, one, *args)
        y8 = oracle.mamba3_step(proj, many, *args, threads=8)
        assert_bitwise(y8, y1, f"threaded step {t}")
    for key in ("ssm", "k_prev", "v_prev"):
        assert_bitwise(many[key], one[key], key)
    assert np.array_equal(many["angle"], one["angle"])


def _mhc_params(rng, n, d, alpha=0.7):
    nw = (rng.random(d) + 0.5).astype(np.float32)
    pw = (rng.standard_normal((2 * n + n * n, d)) * 4 / np.sqrt(d)).astype(np.float32).astype(np.float64)
    pb, qb = rng.standard_normal(n).astype(np.float32), rng.standard_normal(n).astype(np.float32)
    rb = rng.standard_normal((n, n)).astype(np.float32)
    return nw, pw, pb, qb, rb


def test_mhc_invariants(oracle):
    rng = np.random.default_rng(6)
    n, d = 4, 64
    s = rng.standard_normal((1, 30, n, d)).astype(np.float32)
    nw, pw, pb, qb, rb = _mhc_params(rng, n, d)
    agg, pre, post, res = oracle.mhc_prepare(s, nw, 1e-5, pw, pb, qb, rb, 0.7, 0.7, 0.7, 20)
    r = res.astype(np.float64)
    assert np.abs(r.sum(-2) - 1).max() < 1e-6  # columns: exact after the last (column) step
    assert np.abs(r.sum(-1) - 1).max() < 1e-3  # rows: converged
    assert np.all((pre > 0) & (pre < 1)) and np.all((post > 0) & (post < 2))
    # iters = 0 runs one round, like iters = 1.
    r0 = oracle.mhc_prepare(s, nw, 1e-5, pw, pb, qb, rb, 0.7, 0.7, 0.7, 0)[3]
    r1 = oracle.mhc_prepare(s, nw, 1e-5, pw, pb, qb, rb, 0.7, 0.7, 0.7, 1)[3]
    assert_bitwise(r0, r1, "iters 0 == iters 1")
    # alpha = 0: coefficients are the static maps of the biases, for every token.
    _, pre0, post0, res0 = oracle.mhc_prepare(s, nw, 1e-5, pw, pb, qb, rb, 0.0, 0.0, 0.0, 20)
    assert np.allclose(pre0, 1 / (1 + np.exp(-pb.astype(np.float64))), rtol=1e-7)
    assert np.allclose(post0, 2 / (1 + np.exp(-qb.astype(np.float64))), rtol=1e-7)
    m = np.exp(rb.astype(np.float64))
    for _ in range(20):
        m /= m.sum(1, keepdims=True)
        m /= m.sum(0, keepdims=True)
    assert np.allclose(res0, np.broadcast_to(m, res0.shape), rtol=1e-6)
    # n = 1: res = 1.
    nw1, pw1, pb1, qb1, rb1 = _mhc_params(rng, 1, d)
    r_one = oracle.mhc_prepare(s[:, :, :1], nw1, 1e-5, pw1, pb1, qb1, rb1, 0.7, 0.7, 0.7, 5)[3]
    assert np.all(r_one == 1.0)
    # agg = sum_i pre_i s_i exactly rounded from double.
    expect = np.einsum("bln,blnd->bld", pre.astype(np.float64), s.astype(np.float64))
    assert_bitwise(agg, expect.astype(np.float32), "agg")
    # combine closed form in double, one rounding; collapse = mean of rounded streams.
    out = rng.standard_normal((1, 30, d)).astype(np.float32)
    new = oracle.mhc_combine(s, res, post, out)
    e = np.einsum("blij,bljd->blid", res.astype(np.float64), s.astype(np.float64)) + \
        post.astype(np.float64)[..., None] * out.astype(np.float64)[:, :, None, :]
    assert rel_err(new, e) < 1e-7
    col = oracle.mhc_combine(s, res, post, out, collapse=True, materialize=False)
    assert_bitwise(col, new.astype(np.float64).mean(-2).astype(np.float32), "collapse")


def test_mhc_prepare_matches_upstream_logspace_form(oracle):
    """The upstream module's math (mean, RMSNorm, tanh maps, log-space Sinkhorn)
    in fp64 numpy (python/montlok/rdt/reference/Model/layers/mhc.py:40-69,
    146-209): the same fixed point as the oracle's linear-space iteration."""
    rng = np.random.default_rng(8)
    n, d = 4, 32
    s = rng.standard_normal((2, 5, n, d)).astype(np.float32)
    nw, pw, pb, qb, rb = _mhc_params(rng, n, d)
    _, pre, post, res = oracle.mhc_prepare(s, nw, 1e-5, pw, pb, qb, rb, 0.7, 0.6, 0.8, 20)
    m = s.astype(np.float64).mean(-2)
    ref = m / np.sqrt((m ** 2).mean(-1, keepdims=True) + float(np.float32(1e-5))) * nw
    lg = np.tanh(ref @ pw.T)
    assert rel_err(pre, 1 / (1 + np.exp(-(pb + 0.7 * lg[..., :n])))) < 1e-7
    assert rel_err(post, 2 / (1 + np.exp(-(qb + 0.6 * lg[..., n:2 * n])))) < 1e-7
    work = (rb + np.float64(np.float32(0.8)) * lg[..., 2 * n:].reshape(2, 5, n, n))
    for _ in range(20):
        work = work - np.log(np.exp(work).sum(-1, keepdims=True))
        work = work - np.log(np.exp(work).sum(-2, keepdims=True))
    assert rel_err(res, np.exp(work)) < 1e-6


def test_rope_invariants(oracle):
    rng = np.random.default_rng(9)
    B, L, H, hd, nope = 1, 6, 2, 16, 8
    rope = hd - nope
    q = rng.standard_normal((B, L, H, hd)).astype(np.float32)
    kv = rng.standard_normal((B, L, H, nope + hd)).astype(np.float32)
    kr = rng.standard_normal((B, L, rope)).astype(np.float32)
    ang = np.arange(L)[:, None] * (1.0 / 10000 ** (np.arange(0, rope, 2) / rope))[None]
    emb = np.concatenate([ang, ang], 1)
    cos, sin = np.cos(emb).astype(np.float32), np.sin(emb).astype(np.float32)
    qo, ko = oracle.mla_rope(q, kv, kr, cos, sin, nope)
    assert_bitwise(qo[:, 0], q[:, 0], "position 0 identity")
    assert np.array_equal(ko[..., :nope], kv[..., :nope])
    half = rope // 2
    for x, y in ((q[..., nope:], qo[..., nope:]),):
        nx = x[..., :half] ** 2 + x[..., half:] ** 2
        ny = y[..., :half].astype(np.float64) ** 2 + y[..., half:].astype(np.float64) ** 2
        assert np.allclose(nx, ny, rtol=1e-5)
    # Closed form: rotate_half with these tables.
    x1, x2 = kr[..., :half].astype(np.float64), kr[..., half:].astype(np.float64)
    c, s_ = cos.astype(np.float64), sin.astype(np.float64)
    expect = np.concatenate([x1 * c[:, :half] - x2 * s_[:, :half], x2 * c[:, half:] + x1 * s_[:, half:]], -1)
    assert_bitwise(ko[:, :, 0, nope:], expect.astype(np.float32), "k rope")


def test_linear_and_sdpa_against_torch_float64(oracle):
    import torch

    rng = np.random.default_rng(10)
    x = rng.standard_normal((37, 64)).astype(np.float32)
    w = rng.standard_normal((100, 64)).astype(np.float32) / 8
    b = rng.standard_normal(100).astype(np.float32)
    expect = torch.nn.functional.linear(torch.from_numpy(x).double(), torch.from_numpy(w).double(),
                                        torch.from_numpy(b).double()).numpy()
    assert_bitwise(oracle.linear(x, w, b), expect.astype(np.float32), "linear")
    B, L, H, dh = 2, 11, 3, 8
    q, k, v = (rng.standard_normal((B, L, H, dh)).astype(np.float32) for _ in range(3))
    t = [torch.from_numpy(a).double().transpose(1, 2) for a in (q, k, v)]
    for mask, causal in ((0, False), (1, True)):
        e = torch.nn.functional.scaled_dot_product_attention(*t, is_causal=causal, scale=0.3).transpose(1, 2)
        assert rel_err(oracle.sdpa(q, k, v, mask, 0.3), e.numpy()) < 1e-6
    # Trailing queries with a bottom-right causal mask.
    nq = 4
    rows = torch.arange(nq)[:, None] + (L - nq)
    allowed = torch.arange(L)[None, :] <= rows
    e = torch.nn.functional.scaled_dot_product_attention(t[0][:, :, -nq:], t[1], t[2], attn_mask=allowed,
                                                         scale=0.3).transpose(1, 2)
    assert rel_err(oracle.sdpa(q[:, -nq:], k, v, 2, 0.3), e.numpy()) < 1e-6
