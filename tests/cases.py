"""Seeded synthetic inputs for the state codec and FP4 decode tests, in numpy
(oracle side) with torch conversions (device side).  Binary16 arrays are kept
as uint16 bit patterns."""
from __future__ import annotations

import numpy as np

RIDGE_LAYOUTS = ("36_24_68", "16_64_48", "32_32_64", "40_16_72", "24_48_56", "8_80_40", "44_8_76")
TIER_LAYOUTS = ("16_64_48", "8_80_40", "24_48_56", "32_32_64", "36_24_68", "40_16_72", "44_8_76")


def tier_counts(layout):
    a, b, c = map(int, layout.split("_"))
    return a, b, c


def ridge_counts(layout):
    a, b, c = tier_counts(layout)
    return a, b - 4, c + 4


def f16(a):
    return np.asarray(a, dtype=np.float32).astype(np.float16).view(np.uint16)


def f16_to_f32(bits):
    return np.asarray(bits, dtype=np.uint16).view(np.float16).astype(np.float32)


def random_e4m3_bytes(rng, shape):
    """Random finite E4M3FN bytes (no 0x7F / 0xFF)."""
    b = rng.integers(0, 256, size=shape, dtype=np.uint16).astype(np.uint8)
    nan = (b & 0x7F) == 0x7F
    b[nan] ^= 1
    return b


def step_inputs(rng, batch, L, H, P, G, *, x_scale=1.0, d_f32=False, db_f32=False, dt_bias_zero=True,
                bc_scale=1.0, dt_scale=1.0):
    """Inputs of one layer step as in the BASELINE configs: x, B, C, D ~ N(0,1)
    in FP16; raw dt ~ N(0,1) (the kernel applies softplus(dt + dt_bias));
    A = -exp(U(log 1, log 16))."""
    x = f16(rng.standard_normal((batch, L, H, P)) * x_scale)
    dt = f16(rng.standard_normal((batch, L, H)) * dt_scale)
    A = (-np.exp(rng.uniform(np.log(1.0), np.log(16.0), size=H))).astype(np.float32)
    B = f16(rng.standard_normal((batch, L, G, 128)) * bc_scale)
    C = f16(rng.standard_normal((batch, L, G, 128)) * bc_scale)
    D = rng.standard_normal(H).astype(np.float32)
    D = D if d_f32 else f16(D)
    db = np.zeros(H, np.float32) if dt_bias_zero else (rng.standard_normal(H) * 0.5).astype(np.float32)
    db = db if db_f32 else f16(db)
    perm = np.stack([rng.permutation(128) for _ in range(G)]).astype(np.uint8)
    return dict(x=x, dt=dt, A=A, B=B, C=C, D=D, dt_bias=db, perm=perm)


def ridge_statics(rng, G, n8, n4, nz, *, pred_std=0.05, basis_std=0.03, lscale=0.001):
    F = n8 + n4 + 2
    basis = f16(rng.standard_normal((G, nz, 2)) * basis_std)
    ls = f16(np.full((G, 2), lscale, np.float32))
    pred = f16(rng.standard_normal((G, F, nz)) * pred_std)
    return dict(basis=basis, lscale=ls, pred=pred)


def random_packed_state(rng, batch, H, P, n8, n4, *, latent=False, scale_mu=-4.0):
    """Arbitrary packed rows: every byte pattern is a valid carry."""
    rows = (batch, H, P)
    st = dict(
        lo=rng.integers(0, 256, size=rows + (n8 // 2,), dtype=np.uint16).astype(np.uint8),
        hi=rng.integers(0, 256, size=rows + (n8 // 2,), dtype=np.uint16).astype(np.uint8),
        q4=rng.integers(0, 256, size=rows + (n4 // 2,), dtype=np.uint16).astype(np.uint8),
        s8=f16(np.exp(rng.normal(scale_mu, 0.5, size=rows))),
        s4=f16(np.exp(rng.normal(scale_mu + 2.5, 0.5, size=rows))),
    )
    if latent:
        st["latent"] = random_e4m3_bytes(rng, rows + (2,))
    return st


def zero_packed_state(batch, H, P, n8, n4, *, latent=False):
    rows = (batch, H, P)
    st = dict(lo=np.zeros(rows + (n8 // 2,), np.uint8), hi=np.zeros(rows + (n8 // 2,), np.uint8),
              q4=np.zeros(rows + (n4 // 2,), np.uint8), s8=np.zeros(rows, np.uint16), s4=np.zeros(rows, np.uint16))
    if latent:
        st["latent"] = np.zeros(rows + (2,), np.uint8)
    return st


def copy_state(st):
    return {k: v.copy() for k, v in st.items()}


def rel_l2(a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    den = np.sqrt((b * b).sum())
    return float(np.sqrt(((a - b) ** 2).sum()) / (den if den > 0 else 1.0))
