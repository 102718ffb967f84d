"""Write the golden vectors of the RDT4quant kernels from the compiled reference.

Runs the reference's own CPU kernels (rdt4quant_cpu/montlok_*.h, compiled by
oracle/Makefile behind oracle/ref_shim.cpp into oracle/_ref/) on seeded
inputs and stores inputs and outputs as small .npz fixtures next to this
script. Needs the reference checkout (only in the build container):

    make -C oracle ref && python tests/golden/make_golden.py

Shapes follow the reference's own test matrix (rdt4quant_cpu/
montlok_selftest.cpp:948-978 and tests/rdt/test_rdt_kernels.py): vector and
scalar recurrence paths, grouped B/C, odd sizes, iters 0, broadcast streams,
trailing queries.
"""

from __future__ import annotations

import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parents[1]))

from oracle import Reference  # noqa: E402


def f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


def save(name: str, **arrays) -> None:
    np.savez_compressed(HERE / f"{name}.npz", **arrays)


def norms(ref: Reference, rng) -> None:
    cases = {}
    for i, (rows, dim, groups, eps, scale) in enumerate(
            [(37, 256, 1, 1e-6, 3.0), (64, 64, 8, 1e-5, 1.0), (15, 100, 4, 1e-6, 1.0), (9, 12, 3, 1e-5, 2.0)]):
        x = f32(rng.standard_normal((rows, dim)) * scale)
        w = f32(rng.random(dim) + 0.5)
        cases[f"rms{i}_x"], cases[f"rms{i}_w"] = x, w
        cases[f"rms{i}_meta"] = np.array([groups, eps])
        cases[f"rms{i}_out"] = ref.rms_norm(x, w, eps, groups)
        right = f32(rng.standard_normal((rows, dim)))
        cases[f"rms{i}_right"] = right
        cases[f"rms{i}_residual"], cases[f"rms{i}_normalized"] = ref.add_rms_norm(x, right, w, eps, groups)
    for i, (rows, dim, bias) in enumerate([(37, 64, True), (20, 256, False), (11, 66, True)]):
        x = f32(rng.standard_normal((rows, dim)) * 2 + 0.5)
        w = f32(rng.random(dim) + 0.5)
        b = f32(rng.standard_normal(dim) * 0.25) if bias else None
        cases[f"ln{i}_x"], cases[f"ln{i}_w"] = x, w
        if b is not None:
            cases[f"ln{i}_b"] = b
        cases[f"ln{i}_out"] = ref.layer_norm(x, w, b, 1e-5)
    for i, (rows, hidden) in enumerate([(37, 100), (8, 51)]):
        x = f32(rng.standard_normal((rows, 2 * hidden)) * 2)
        cases[f"swiglu{i}_x"] = x
        cases[f"swiglu{i}_out"] = ref.swiglu(x)
    save("norms", **cases)


def siso(ref: Reference, rng) -> None:
    cases = {}
    # (B, L, H, N, D): 16-lane blocks, 8-lane blocks, scalar path, odd N.
    for i, (B, L, H, N, D) in enumerate([(2, 24, 4, 16, 32), (1, 19, 3, 14, 8), (2, 11, 2, 6, 12),
                                         (1, 9, 2, 7, 16)]):
        q = f32(rng.standard_normal((B, L, H, N)) * 0.5)
        k = f32(rng.standard_normal((B, L, H, N)) * 0.5)
        v = f32(rng.standard_normal((B, L, H, D)))
        z = f32(rng.standard_normal((B, L, H, D)) * 3)
        dt = np.log1p(np.exp(f32(rng.standard_normal((B, L, H)) - 2.0))).astype(np.float32)
        adt = f32(-(np.abs(rng.standard_normal((B, L, H))) + 0.5) * dt)
        trap = f32(rng.standard_normal((B, L, H)))
        skip = f32(rng.standard_normal(H))
        al, be, ga = ref.step_coefficients(adt, dt, trap)
        gate = f32(z / (1.0 + np.exp(-z.astype(np.float64))))
        for key, val in dict(q=q, k=k, v=v, z=z, adt=adt, dt=dt, trap=trap, skip=skip, alpha=al, beta=be, gamma=ga,
                             gate=gate).items():
            cases[f"c{i}_{key}"] = val
        cases[f"c{i}_out"] = ref.siso(q, k, v, gate, al, be, ga, skip, gate_logits=False)
        cases[f"c{i}_out_silu"] = ref.siso(q, k, v, z, al, be, ga, skip, gate_logits=True)
    save("siso", **cases)


def mamba_forward(ref: Reference, rng) -> None:
    cases = {}
    # (B, L, N, G, H, D, R): rope 4/3/1/0 angles, 2 B/C groups, scalar headdim.
    for i, (B, L, N, G, H, D, R) in enumerate([(2, 24, 16, 1, 4, 16, 4), (1, 19, 14, 2, 4, 8, 3),
                                               (1, 13, 6, 1, 3, 12, 1), (1, 7, 8, 1, 2, 8, 0),
                                               (1, 32, 64, 1, 2, 64, 16)]):
        W = 2 * H * D + 2 * G * N + 3 * H + R
        proj = f32(rng.standard_normal((B, L, W)))
        bb = f32(1 + 0.3 * rng.standard_normal((H, N)))
        cb = f32(1 + 0.3 * rng.standard_normal((H, N)))
        bw = f32(rng.random(N) + 0.5)
        cw = f32(rng.random(N) + 0.5)
        dtb = f32(rng.standard_normal(H) - 2.0)
        skip = f32(rng.standard_normal(H) * 0.5 + 1.0)
        geom = (N, G, H, D, R)
        args = (bb, cb, bw, cw, 1e-5, 1e-5, dtb)
        qv, kv, al, be, ga = ref.prep(proj, *geom, *args, 1e-4)
        out = ref.mamba3_siso_forward(proj, *geom, *args, skip, 1e-4)
        for key, val in dict(proj=proj, b_bias=bb, c_bias=cb, b_norm_w=bw, c_norm_w=cw, dt_bias=dtb, skip=skip,
                             q=qv, k=kv, alpha=al, beta=be, gamma=ga, out=out).items():
            cases[f"c{i}_{key}"] = val
        cases[f"c{i}_geom"] = np.array(geom, dtype=np.int64)
    save("mamba_forward", **cases)


def mhc(ref: Reference, rng) -> None:
    cases = {}
    # (n, d, B, L, iters): model n, odd d, iters 0, n = 1, n = 9 (montlok_selftest.cpp:948-978 spirit).
    for i, (n, d, B, L, iters) in enumerate([(4, 128, 1, 24, 20), (4, 256, 2, 9, 20), (3, 100, 1, 10, 5),
                                             (5, 33, 2, 7, 0), (1, 16, 1, 9, 3), (9, 20, 1, 6, 2)]):
        s = f32(rng.standard_normal((B, L, n, d)) * 1.5)
        nw = f32(rng.random(d) + 0.5)
        pw = (f32(rng.standard_normal((2 * n + n * n, d)) * 4 / np.sqrt(d))).astype(np.float64)
        pb = f32(rng.standard_normal(n) * 0.5 + np.log(1.0 / max(n - 1, 1)))
        qb = f32(rng.standard_normal(n) * 0.5)
        rb = f32(np.eye(n) * 3.0 + rng.standard_normal((n, n)))
        anw = f32(rng.random(d) + 0.5)
        params = (nw, 1e-5, pw, pb, qb, rb, 0.7, 0.6, 0.8, iters)
        agg, pre, post, res = ref.mhc_prepare(s, *params)
        agg_n = ref.mhc_prepare(s, *params, 0, anw, 1e-6)[0]
        back = f32(s[:, :, 0, :])
        b_out = ref.mhc_prepare(back, *params, n)
        out = f32(np.tanh(agg))
        new = ref.mhc_combine(s, res, post, out)
        col = ref.mhc_combine(s, res, post, out, collapse=True, materialize=False)
        nxt = ref.mhc_combine_prepare(s, res, post, out, *params)
        for key, val in dict(streams=s, norm_w=nw, proj_w=pw, pre_bias=pb, post_bias=qb, res_bias=rb, agg_norm_w=anw,
                             agg=agg, pre=pre, post=post, res=res, agg_normed=agg_n, bcast_agg=b_out[0],
                             bcast_pre=b_out[1], bcast_post=b_out[2], bcast_res=b_out[3], out=out, new=new,
                             collapsed=col, next_new=nxt[0], next_agg=nxt[1], next_pre=nxt[2], next_post=nxt[3],
                             next_res=nxt[4]).items():
            cases[f"c{i}_{key}"] = val
        cases[f"c{i}_meta"] = np.array([n, d, iters], dtype=np.int64)
    cases["alphas"] = np.array([0.7, 0.6, 0.8], dtype=np.float32)
    save("mhc", **cases)


def rope(ref: Reference, rng) -> None:
    cases = {}
    for i, (B, L, H, hd, nope, q_len) in enumerate([(2, 13, 4, 64, 32, 13), (1, 17, 8, 32, 16, 17),
                                                    (2, 9, 2, 16, 0, 9), (2, 13, 4, 64, 32, 5),
                                                    (1, 7, 3, 24, 16, 1)]):
        rope_dim = hd - nope
        q = f32(rng.standard_normal((B, q_len, H, hd)))
        kv = f32(rng.standard_normal((B, L, H, nope + hd)))
        kr = f32(rng.standard_normal((B, L, rope_dim)))
        inv_freq = 1.0 / (10000.0 ** (np.arange(0, rope_dim, 2, dtype=np.float32) / rope_dim))
        ang = np.arange(L, dtype=np.float32)[:, None] * inv_freq[None, :].astype(np.float32)
        emb = np.concatenate([ang, ang], 1).astype(np.float32)
        cos, sin = f32(np.cos(emb)), f32(np.sin(emb))
        q_out, k_out = ref.mla_rope(q, kv, kr, cos, sin, nope)
        for key, val in dict(q=q, kv=kv, k_rope=kr, cos=cos, sin=sin, q_out=q_out, k_out=k_out).items():
            cases[f"c{i}_{key}"] = val
        cases[f"c{i}_nope"] = np.array([nope], dtype=np.int64)
    save("rope", **cases)


def main() -> None:
    ref = Reference("avx2")
    ref.set_threads(1)
    norms(ref, np.random.default_rng(13))
    siso(ref, np.random.default_rng(7))
    mamba_forward(ref, np.random.default_rng(11))
    mhc(ref, np.random.default_rng(23))
    rope(ref, np.random.default_rng(41))
    total = sum(p.stat().st_size for p in HERE.glob("*.npz"))
    print(f"golden fixtures written: {sorted(p.name for p in HERE.glob('*.npz'))}, {total} bytes")


if __name__ == "__main__":
    main()
