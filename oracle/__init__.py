"""CPU oracle for the RDT4quant fused-forward path (test infrastructure only).

Two CPU implementations behind one numpy-level API:

* ``Oracle``    -- this repository's C restatement (``oracle/mlk_oracle.c``),
                   built into ``oracle/_build/libmlk_oracle.so``.
* ``Reference`` -- the reference's own header-only kernels
                   (rdt4quant_cpu/montlok_*.h) compiled behind ``ref_shim.cpp``
                   into ``oracle/_ref/``; present only where the reference
                   checkout was available when ``oracle/Makefile`` ran.

Only tests, ``__graft_entry__.smoke()`` and the cpu_baseline leg of
``bench.py`` may import this package, and only to check results or as the
timed CPU baseline. The product path never routes through it.
"""

from __future__ import annotations

import ctypes as C
import os
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
ORACLE_LIB = HERE / "_build" / "libmlk_oracle.so"
REF_DIR = HERE / "_ref"

_f32p = C.POINTER(C.c_float)
_f64p = C.POINTER(C.c_double)
_i64p = C.POINTER(C.c_int64)
_i64 = C.c_int64
_dbl = C.c_double


def build(quiet: bool = True) -> None:
    """Compile the oracle (and the reference shim when the reference exists)."""
    out = subprocess.run(["make", "-C", str(HERE), "all"], capture_output=True, text=True)
    if out.returncode != 0:
        raise RuntimeError(f"oracle build failed:\n{out.stdout}\n{out.stderr}")
    if not quiet:
        print(out.stdout)


def _f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


def _ptr(a: np.ndarray | None, kind=_f32p):
    if a is None:
        return None
    return a.ctypes.data_as(kind)


def _strides(s) -> np.ndarray:
    return np.ascontiguousarray(np.asarray(s, dtype=np.int64))


def host_isa() -> str:
    """'avx512' when the host has AVX-512 F/BW/DQ/VL, else 'avx2'."""
    try:
        flags = Path("/proc/cpuinfo").read_text()
    except OSError:
        return "avx2"
    need = ("avx512f", "avx512bw", "avx512dq", "avx512vl")
    return "avx512" if all(f" {flag}" in flags for flag in need) else "avx2"


class _Lib:
    prefix = ""

    def __init__(self, path: Path):
        self.path = path
        self.lib = C.CDLL(str(path))
        self._declare()

    def _fn(self, name):
        return getattr(self.lib, self.prefix + name)

    def _declare(self):
        p = self.prefix
        L = self.lib
        getattr(L, p + "rms_norm").argtypes = [_f32p, _i64, _f32p, _dbl, _i64, _i64, _i64, _f32p]
        getattr(L, p + "add_rms_norm").argtypes = [_f32p, _f32p, _f32p, _dbl, _i64, _i64, _i64, _f32p, _f32p]
        getattr(L, p + "layer_norm").argtypes = [_f32p, _i64, _f32p, _f32p, _dbl, _i64, _i64, _f32p]
        getattr(L, p + "swiglu").argtypes = [_f32p, _i64, _i64, _i64, _f32p]
        getattr(L, p + "step_coefficients").argtypes = [_f32p, _f32p, _f32p, _i64, _f32p, _f32p, _f32p]
        getattr(L, p + "siso").argtypes = [_i64] * 5 + [_f32p, _i64p] * 4 + [C.c_int] + [_f32p] * 5 + [_i64p]
        mhc_prep = [_f32p, _i64, _i64, _f32p, _dbl, _f64p, _f32p, _f32p, _f32p, C.c_float, C.c_float, C.c_float,
                    _i64, _i64, _i64, _i64, _f32p, _dbl, _f32p, _f32p, _f32p, _f32p]
        getattr(L, p + "mhc_prepare").argtypes = mhc_prep

    # ---------------------------------------------------------------- norms
    def rms_norm(self, x, w, eps, groups=1):
        x = _f32(x)
        dim = x.shape[-1]
        rows = x.size // dim
        out = np.empty_like(x)
        self._fn("rms_norm")(_ptr(x), dim, _ptr(_f32(w)), eps, dim, groups, rows, _ptr(out))
        return out

    def add_rms_norm(self, left, right, w, eps, groups=1):
        left, right = _f32(left), _f32(right)
        dim = left.shape[-1]
        rows = left.size // dim
        residual = np.empty_like(left)
        normalized = np.empty_like(left)
        self._fn("add_rms_norm")(_ptr(left), _ptr(right), _ptr(_f32(w)), eps, dim, groups, rows, _ptr(residual),
                                 _ptr(normalized))
        return residual, normalized

    def layer_norm(self, x, w, bias, eps):
        x = _f32(x)
        dim = x.shape[-1]
        rows = x.size // dim
        out = np.empty_like(x)
        b = None if bias is None else _f32(bias)
        self._fn("layer_norm")(_ptr(x), dim, _ptr(_f32(w)), _ptr(b), eps, dim, rows, _ptr(out))
        return out

    def swiglu(self, x):
        x = _f32(x)
        width = x.shape[-1]
        hidden = width // 2
        rows = x.size // width
        out = np.empty(x.shape[:-1] + (hidden,), dtype=np.float32)
        self._fn("swiglu")(_ptr(x), width, hidden, rows, _ptr(out))
        return out

    # ---------------------------------------------------------------- mamba
    def step_coefficients(self, adt, dt, trap):
        adt, dt, trap = _f32(adt), _f32(dt), _f32(trap)
        alpha, beta, gamma = (np.empty_like(adt) for _ in range(3))
        self._fn("step_coefficients")(_ptr(adt), _ptr(dt), _ptr(trap), adt.size, _ptr(alpha), _ptr(beta),
                                      _ptr(gamma))
        return alpha, beta, gamma

    def siso(self, q, k, v, gate, alpha, beta, gamma, skip, gate_logits=False):
        """Recurrence over contiguous q,k [B,L,H,N], v,gate [B,L,H,D]."""
        q, k, v, gate = _f32(q), _f32(k), _f32(v), _f32(gate)
        B, L, H, N = q.shape
        D = v.shape[-1]
        out = np.empty((B, L, H, D), dtype=np.float32)
        qs = _strides([L * H * N, H * N, N])
        vs = _strides([L * H * D, H * D, D])
        self._fn("siso")(B, L, H, N, D, _ptr(q), _ptr(qs, _i64p), _ptr(k), _ptr(qs, _i64p), _ptr(v),
                         _ptr(vs, _i64p), _ptr(gate), _ptr(vs, _i64p), int(gate_logits), _ptr(_f32(alpha)),
                         _ptr(_f32(beta)), _ptr(_f32(gamma)), _ptr(_f32(skip)), _ptr(out), _ptr(vs, _i64p))
        return out

    # ---------------------------------------------------------------- mHC
    def mhc_prepare(self, streams, norm_w, eps, proj_w64, pre_bias, post_bias, res_bias, pre_alpha, post_alpha,
                    res_alpha, iters, n_streams=0, agg_norm_w=None, agg_norm_eps=0.0):
        """streams [B,L,n,d] or broadcast [B,L,d] (n_streams required)."""
        streams = _f32(streams)
        if streams.ndim == 4:
            B, L, n, d = streams.shape
            sd, ts = d, n * d
        else:
            B, L, d = streams.shape
            n = n_streams
            sd, ts = 0, d
        T = B * L
        agg = np.empty((B, L, d), np.float32)
        pre = np.empty((B, L, n), np.float32)
        post = np.empty((B, L, n), np.float32)
        res = np.empty((B, L, n, n), np.float32)
        w64 = np.ascontiguousarray(proj_w64, dtype=np.float64)
        anw = None if agg_norm_w is None else _f32(agg_norm_w)
        self._fn("mhc_prepare")(_ptr(streams), sd, ts, _ptr(_f32(norm_w)), eps, _ptr(w64, _f64p),
                                _ptr(_f32(pre_bias)), _ptr(_f32(post_bias)), _ptr(_f32(res_bias)), float(pre_alpha),
                                float(post_alpha), float(res_alpha), iters, T, n, d, _ptr(anw), agg_norm_eps,
                                _ptr(agg), _ptr(pre), _ptr(post), _ptr(res))
        return agg, pre, post, res


class Oracle(_Lib):
    prefix = "orc_"

    def __init__(self, path: Path = ORACLE_LIB):
        if not path.exists():
            build()
        super().__init__(path)
        L = self.lib
        L.orc_prep.argtypes = [_i64, _i64, _f32p, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _f32p, _f32p, _f32p,
                               _f32p, _dbl, _dbl, _f32p, _dbl, _f32p, _f32p, _f32p, _f32p, _f32p]
        L.orc_mamba3_siso_forward.argtypes = [_i64, _i64, _f32p, _i64, _i64] + [_i64] * 5 + [_f32p] * 4 + [
            _dbl, _dbl, _f32p, _f32p, _dbl, _f32p]
        L.orc_mamba3_step.argtypes = [_i64, _f32p, _i64] + [_i64] * 5 + [_f32p] * 4 + [_dbl, _dbl, _f32p, _f32p,
                                                                                      _dbl, _f32p, _f32p, _f32p,
                                                                                      _f64p, C.c_int, _f32p]
        L.orc_mamba3_step_threads.argtypes = [C.c_int] + L.orc_mamba3_step.argtypes
        L.orc_mhc_combine.argtypes = [_f32p, _i64, _i64, _f32p, _f32p, _f32p, _i64, _i64, _i64, _f32p, _f32p]
        L.orc_mla_rope.argtypes = [_f32p, _i64, _i64, _f32p, _f32p, _i64, _f32p, _f32p, _f32p] + [_i64] * 5
        L.orc_linear.argtypes = [_f32p, _i64, _f32p, _f32p, _i64, _i64, _i64, _f32p]
        L.orc_sdpa.argtypes = [_f32p, _i64, _f32p, _i64, _f32p, _i64] + [_i64] * 5 + [C.c_int, _dbl, _f32p]

    def prep(self, proj, N, G, H, D, R, b_bias, c_bias, b_norm_w, c_norm_w, b_eps, c_eps, dt_bias, a_floor):
        proj = _f32(proj)
        B, L, W = proj.shape
        q = np.empty((B, L, H, N), np.float32)
        k = np.empty_like(q)
        alpha, beta, gamma = (np.empty((B, L, H), np.float32) for _ in range(3))
        self.lib.orc_prep(B, L, _ptr(proj), L * W, W, H * D, N, G, H, R, _ptr(_f32(b_bias)), _ptr(_f32(c_bias)),
                          _ptr(_f32(b_norm_w)), _ptr(_f32(c_norm_w)), b_eps, c_eps, _ptr(_f32(dt_bias)), a_floor,
                          _ptr(q), _ptr(k), _ptr(alpha), _ptr(beta), _ptr(gamma))
        return q, k, alpha, beta, gamma

    def mamba3_siso_forward(self, proj, N, G, H, D, R, b_bias, c_bias, b_norm_w, c_norm_w, b_eps, c_eps, dt_bias,
                            skip, a_floor):
        proj = _f32(proj)
        B, L, W = proj.shape
        out = np.empty((B, L, H * D), np.float32)
        self.lib.orc_mamba3_siso_forward(B, L, _ptr(proj), L * W, W, N, G, H, D, R, _ptr(_f32(b_bias)),
                                         _ptr(_f32(c_bias)), _ptr(_f32(b_norm_w)), _ptr(_f32(c_norm_w)), b_eps, c_eps,
                                         _ptr(_f32(dt_bias)), _ptr(_f32(skip)), a_floor, _ptr(out))
        return out

    def mamba3_step(self, proj, state, N, G, H, D, R, b_bias, c_bias, b_norm_w, c_norm_w, b_eps, c_eps, dt_bias,
                    skip, a_floor, threads=1):
        """One token for S streams; `state` = dict(ssm, k_prev, v_prev, angle, started) updated in place.
        threads > 1 splits the streams over that many OpenMP threads (same result)."""
        proj = _f32(proj)
        S, W = proj.shape
        out = np.empty((S, H * D), np.float32)
        for key, dtype in (("ssm", np.float32), ("k_prev", np.float32), ("v_prev", np.float32),
                           ("angle", np.float64)):
            assert state[key].dtype == dtype and state[key].flags.c_contiguous, key
        fn = self.lib.orc_mamba3_step if threads <= 1 else \
            (lambda *a: self.lib.orc_mamba3_step_threads(int(threads), *a))
        fn(S, _ptr(proj), W, N, G, H, D, R, _ptr(_f32(b_bias)), _ptr(_f32(c_bias)),
                                 _ptr(_f32(b_norm_w)), _ptr(_f32(c_norm_w)), b_eps, c_eps, _ptr(_f32(dt_bias)),
                                 _ptr(_f32(skip)), a_floor, _ptr(state["ssm"]), _ptr(state["k_prev"]),
                                 _ptr(state["v_prev"]), _ptr(state["angle"], _f64p), int(state["started"]),
                                 _ptr(out))
        state["started"] = 1
        return out

    def mhc_combine(self, streams, res, post, out, collapse=False, materialize=True):
        streams = _f32(streams)
        res, post, out = _f32(res), _f32(post), _f32(out)
        B, L, n = post.shape
        d = out.shape[-1]
        sd, ts = (d, n * d) if streams.ndim == 4 else (0, d)
        new = np.empty((B, L, n, d), np.float32) if materialize else None
        col = np.empty((B, L, d), np.float32) if collapse else None
        self.lib.orc_mhc_combine(_ptr(streams), sd, ts, _ptr(res), _ptr(post), _ptr(out), B * L, n, d, _ptr(new),
                                 _ptr(col))
        if collapse and not materialize:
            return col
        if collapse:
            return new, col
        return new

    def mla_rope(self, q, kv, k_rope, cos, sin, nope_dim):
        """q [B,Lq,H,hd] (copied, rotated copy returned), kv [B,L,H,nope+hd], k_rope [B,L,rope]."""
        q = _f32(q).copy()
        kv, k_rope, cos, sin = _f32(kv), _f32(k_rope), _f32(cos), _f32(sin)
        B, Lq, H, hd = q.shape
        L = kv.shape[1]
        k = np.empty((B, L, H, hd), np.float32)
        self.lib.orc_mla_rope(_ptr(q), H * hd, Lq, _ptr(kv), _ptr(k_rope), k_rope.shape[-1], _ptr(cos), _ptr(sin),
                              _ptr(k), B, L, H, hd, nope_dim)
        return q, k

    def linear(self, x, w, bias=None):
        x = _f32(x)
        K = x.shape[-1]
        M = x.size // K
        w = _f32(w)
        N = w.shape[0]
        out = np.empty(x.shape[:-1] + (N,), np.float32)
        self.lib.orc_linear(_ptr(x), K, _ptr(w), _ptr(None if bias is None else _f32(bias)), M, K, N, _ptr(out))
        return out

    def sdpa(self, q, k, v, mask, scale):
        """q [B,Lq,H,dh], k/v [B,Lk,H,dh]; mask 0 none, 1 top-left causal, 2 bottom-right causal."""
        q, k, v = _f32(q), _f32(k), _f32(v)
        B, Lq, H, dh = q.shape
        Lk = k.shape[1]
        out = np.empty((B, Lq, H, dh), np.float32)
        self.lib.orc_sdpa(_ptr(q), H * dh, _ptr(k), H * dh, _ptr(v), H * dh, B, H, Lq, Lk, dh, mask, scale,
                          _ptr(out))
        return out


class Reference(_Lib):
    prefix = "ref_"

    def __init__(self, variant: str | None = None):
        variant = variant or host_isa()
        path = REF_DIR / f"libmlk_ref_{variant}.so"
        if not path.exists():
            raise FileNotFoundError(f"{path} is not built (oracle/Makefile needs the reference checkout)")
        super().__init__(path)
        self.variant = variant
        L = self.lib
        L.ref_set_threads.argtypes = [C.c_int]
        L.ref_max_threads.restype = C.c_int
        L.ref_vec_bytes.restype = C.c_int
        L.ref_prep.argtypes = [_i64, _i64, _i64, _f32p, _i64, _i64] + [_i64] * 6 + [_f32p] * 4 + [
            _dbl, _dbl, _f32p, _dbl] + [_f32p] * 7
        L.ref_mamba3_siso_forward.argtypes = [_i64, _i64, _f32p, _i64, _i64] + [_i64] * 5 + [_f32p] * 4 + [
            _dbl, _dbl, _f32p, _f32p, _dbl] + [_f32p] * 6
        L.ref_mhc_combine.argtypes = [_f32p, _i64, _i64, _f32p, _f32p, _f32p, _i64, _i64, _i64, _f32p, _f32p,
                                      C.c_int]
        L.ref_mhc_combine_prepare.argtypes = [_f32p, _i64, _i64, _f32p, _f32p, _f32p, _f32p, _dbl, _f64p, _f32p,
                                              _f32p, _f32p, C.c_float, C.c_float, C.c_float, _i64, _i64, _i64, _i64,
                                              _f32p, _dbl] + [_f32p] * 5
        L.ref_mla_rope.argtypes = [_f32p, _i64, _i64, _i64, _f32p, _i64, _i64, _f32p, _i64, _f32p, _f32p, _f32p] + [
            _i64] * 5

    def set_threads(self, threads: int) -> None:
        self.lib.ref_set_threads(int(threads))

    def max_threads(self) -> int:
        return int(self.lib.ref_max_threads())

    def prep(self, proj, N, G, H, D, R, b_bias, c_bias, b_norm_w, c_norm_w, b_eps, c_eps, dt_bias, a_floor):
        proj = _f32(proj)
        B, L, W = proj.shape
        Rw = max(R, 1)
        q = np.empty((B, L, H, N), np.float32)
        k = np.empty_like(q)
        alpha, beta, gamma = (np.empty((B, L, H), np.float32) for _ in range(3))
        term = np.empty(B * L * H * Rw, np.float32)
        cum = np.empty(B * L * H * Rw, np.float32)
        self.lib.ref_prep(B, L, W, _ptr(proj), L * W, W, H * D, N, G, H, D, R, _ptr(_f32(b_bias)),
                          _ptr(_f32(c_bias)), _ptr(_f32(b_norm_w)), _ptr(_f32(c_norm_w)), b_eps, c_eps,
                          _ptr(_f32(dt_bias)), a_floor, _ptr(q), _ptr(k), _ptr(alpha), _ptr(beta), _ptr(gamma),
                          _ptr(term), _ptr(cum))
        return q, k, alpha, beta, gamma

    def mamba3_siso_forward(self, proj, N, G, H, D, R, b_bias, c_bias, b_norm_w, c_norm_w, b_eps, c_eps, dt_bias,
                            skip, a_floor):
        proj = _f32(proj)
        B, L, W = proj.shape
        Rw = max(R, 1)
        q = np.empty(B * L * H * N, np.float32)
        k = np.empty_like(q)
        coef = np.empty(3 * B * L * H, np.float32)
        term = np.empty(B * L * H * Rw, np.float32)
        cum = np.empty_like(term)
        out = np.empty((B, L, H * D), np.float32)
        self.lib.ref_mamba3_siso_forward(B, L, _ptr(proj), L * W, W, N, G, H, D, R, _ptr(_f32(b_bias)),
                                         _ptr(_f32(c_bias)), _ptr(_f32(b_norm_w)), _ptr(_f32(c_norm_w)), b_eps, c_eps,
                                         _ptr(_f32(dt_bias)), _ptr(_f32(skip)), a_floor, _ptr(q), _ptr(k),
                                         _ptr(coef), _ptr(term), _ptr(cum), _ptr(out))
        return out

    def mhc_combine(self, streams, res, post, out, collapse=False, materialize=True):
        streams = _f32(streams)
        res, post, out = _f32(res), _f32(post), _f32(out)
        B, L, n = post.shape
        d = out.shape[-1]
        sd, ts = (d, n * d) if streams.ndim == 4 else (0, d)
        if collapse and not materialize:
            col = np.empty((B, L, d), np.float32)
            self.lib.ref_mhc_combine(_ptr(streams), sd, ts, _ptr(res), _ptr(post), _ptr(out), B * L, n, d, None,
                                     _ptr(col), 1)
            return col
        new = np.empty((B, L, n, d), np.float32)
        col = np.empty((B, L, d), np.float32) if collapse else None
        self.lib.ref_mhc_combine(_ptr(streams), sd, ts, _ptr(res), _ptr(post), _ptr(out), B * L, n, d, _ptr(new),
                                 _ptr(col), 0)
        return (new, col) if collapse else new

    def mhc_combine_prepare(self, streams, res, post, out, norm_w, eps, proj_w64, pre_bias, post_bias, res_bias,
                            pre_alpha, post_alpha, res_alpha, iters, agg_norm_w=None, agg_norm_eps=0.0):
        streams = _f32(streams)
        res, post, out = _f32(res), _f32(post), _f32(out)
        B, L, n = post.shape
        d = out.shape[-1]
        sd, ts = (d, n * d) if streams.ndim == 4 else (0, d)
        new = np.empty((B, L, n, d), np.float32)
        agg = np.empty((B, L, d), np.float32)
        pre_o = np.empty((B, L, n), np.float32)
        post_o = np.empty((B, L, n), np.float32)
        res_o = np.empty((B, L, n, n), np.float32)
        w64 = np.ascontiguousarray(proj_w64, dtype=np.float64)
        anw = None if agg_norm_w is None else _f32(agg_norm_w)
        self.lib.ref_mhc_combine_prepare(_ptr(streams), sd, ts, _ptr(res), _ptr(post), _ptr(out), _ptr(_f32(norm_w)),
                                         eps, _ptr(w64, _f64p), _ptr(_f32(pre_bias)), _ptr(_f32(post_bias)),
                                         _ptr(_f32(res_bias)), float(pre_alpha), float(post_alpha), float(res_alpha),
                                         iters, B * L, n, d, _ptr(anw), agg_norm_eps, _ptr(new), _ptr(agg),
                                         _ptr(pre_o), _ptr(post_o), _ptr(res_o))
        return new, agg, pre_o, post_o, res_o

    def mla_rope(self, q, kv, k_rope, cos, sin, nope_dim):
        q = _f32(q).copy()
        kv, k_rope, cos, sin = _f32(kv), _f32(k_rope), _f32(cos), _f32(sin)
        B, Lq, H, hd = q.shape
        L = kv.shape[1]
        k = np.empty((B, L, H, hd), np.float32)
        self.lib.ref_mla_rope(_ptr(q), H * hd, hd, Lq, _ptr(kv), H * (nope_dim + hd), nope_dim + hd, _ptr(k_rope),
                              k_rope.shape[-1], _ptr(cos), _ptr(sin), _ptr(k), B, L, H, hd, nope_dim)
        return q, k


def reference_available(variant: str | None = None) -> bool:
    variant = variant or host_isa()
    return (REF_DIR / f"libmlk_ref_{variant}.so").exists()
