"""Pins of the CPU oracle: every golden vector and known-answer check the
reference holds for this path, library routines (numpy binary16, torch
float8_e4m3fn), closed forms and invariants.  Each check is chosen so that a
plausible restatement mistake fails it."""
import json
import math
from pathlib import Path

import numpy as np
import pytest
import torch

import cases

GOLDEN = Path(__file__).resolve().parent / "golden"


# ---------------------------------------------------------------- formats

def test_f16_decode_every_pattern_matches_numpy(oracle):
    every = np.arange(65536, dtype=np.uint32)
    got = oracle.unary(every, 1).view(np.float32)
    want = every.astype(np.uint16).view(np.float16).astype(np.float32)
    same = (got.view(np.uint32) == want.view(np.uint32)) | (np.isnan(got) & np.isnan(want))
    assert same.all()


def test_f16_encode_matches_numpy_rne(oracle):
    rng = np.random.default_rng(0)
    f = np.arange(65536, dtype=np.uint16).view(np.float16).astype(np.float32)
    f = np.sort(f[np.isfinite(f)])
    mids = ((f[:-1].astype(np.float64) + f[1:]) / 2).astype(np.float32)   # ties: exactly representable
    vals = np.concatenate([f, mids, np.nextafter(mids, np.inf), np.nextafter(mids, -np.inf),
                           rng.standard_normal(1 << 18).astype(np.float32) * 1e4,
                           np.float32([65519.99, 65520.0, 7e4, 1e-8, 2.98e-8, 3e-8, -0.0])])
    got = oracle.unary(vals.view(np.uint32), 0).astype(np.uint16)
    with np.errstate(over="ignore"):
        want = vals.astype(np.float16).view(np.uint16)
    assert (got == want).all()


def test_e4m3_reference_kat(oracle):
    """docs/evidence/fp_state_diagnostics/v13/cpu_reference.json: 254 finite
    E4M3FN bit patterns with 253 unique values (+0 and -0)."""
    kat = json.loads((GOLDEN / "v13_cpu_reference_checks.json").read_text())
    vals = oracle.unary(np.arange(256, dtype=np.uint32), 3).view(np.float32)
    finite = np.isfinite(vals)
    assert int(finite.sum()) == kat["fp8_finite_bit_patterns"] == 254
    assert len(set(vals[finite].tolist())) == kat["fp8_unique_values"] == 253


def test_e4m3_matches_torch_float8(oracle):
    every = np.arange(256, dtype=np.uint8)
    want = torch.from_numpy(every).view(torch.float8_e4m3fn).float().numpy()
    got = oracle.unary(every.astype(np.uint32), 3).view(np.float32)
    assert ((got == want) | (np.isnan(got) & np.isnan(want))).all()
    assert (np.signbit(got[every != 0x7F]) == np.signbit(want[every != 0x7F])).all()
    # encode: every representable value, every midpoint and its neighbours,
    # random values in the clamp range
    f = np.sort(np.unique(want[np.isfinite(want)]))
    mids = ((f[:-1].astype(np.float64) + f[1:]) / 2).astype(np.float32)
    rng = np.random.default_rng(1)
    vals = np.concatenate([f, mids, np.nextafter(mids, np.inf), np.nextafter(mids, -np.inf),
                           rng.uniform(-448, 448, 1 << 18).astype(np.float32),
                           rng.uniform(-0.03, 0.03, 1 << 16).astype(np.float32), np.float32([-0.0, 0.0])])
    got = oracle.unary(vals.view(np.uint32), 2).astype(np.uint8)
    want = torch.from_numpy(vals).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    assert (got == want).all()


def test_fp4_tie_kat_reference_encoder_rule():
    """v13/cpu_reference.json: E2M1 ties [.25,.75,1.25,1.75,2.5,3.5,5] go to the
    even codes [0,2,2,4,4,6,6]; the decode table is the reference's
    E2M1_MAGNITUDES.  (Pins the magnitude table the decoder uses.)"""
    kat = json.loads((GOLDEN / "v13_cpu_reference_checks.json").read_text())
    lev = [0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0]
    for tie, code in zip(kat["fp4_ties"], kat["fp4_even_codes"]):
        lo = max(i for i, v in enumerate(lev) if v < tie)
        assert tie == (lev[lo] + lev[lo + 1]) / 2 and code in (lo, lo + 1) and code % 2 == 0


# --------------------------------------------------------- rounding identities

def test_round_half_away_identity_exhaustive(oracle):
    """trunc(x + copysign(pred(0.5), x)) == roundf(x) for every binary32 with
    |x| < 2^25 (both signs): the device quantizer's rounding."""
    assert oracle.check_round_identity(0, 0x4C000000) == 0


def test_reciprocal_quantizer_equals_ieee_division(oracle):
    codes_bad, div_bad = oracle.check_markstein(20260901, 50_000_000, 3000)
    assert codes_bad == 0 and div_bad == 0


def test_latent_reciprocal_division_gives_ieee_e4m3_bytes(oracle):
    """Every binary16 latent scale: copysign(reciprocal-form quotient, z)
    yields the same E4M3 byte as IEEE z / ls, signed zeros and subnormals
    included."""
    assert oracle.check_latent_division(77, 400) == 0


def test_stored_quantize_kat(oracle):
    """state_ppl_codec_v6.py:54-61: exact half ties go away from zero, a zero
    or underflowed scale gives 0, codes clamp at +-limit."""
    s = cases.f16([0.5, 0.5, 0.5, 0.5, 1.0, 1e-8, 0.0, 2.0 ** -24, 0.25])
    v = np.float32([1.75, -1.75, 1.25, 100.0, 3.5, 5.0, 3.0, 127.5 * 2.0 ** -24, -0.125])
    q = oracle.stored_quantize(v, s, 7)
    assert q.tolist() == [4, -4, 3, 7, 4, 0, 0, 7, -1]   # 3.5 -> 4, -3.5 -> -4, 2.5 -> 3
    q = oracle.stored_quantize(np.float32([127.5 * 2.0 ** -24, -126.5 * 0.5]), cases.f16([2.0 ** -24, 0.5]), 127)
    assert q.tolist() == [127, -127]


# ------------------------------------------------------------ transcendentals

def test_exp_log_recipe_matches_correctly_rounded_libm(oracle):
    """The codec's exp/log recipe equals binary32 rounding of libm's
    binary64 results (which are within 1 ulp of exact) on a dense sample."""
    rng = np.random.default_rng(2)
    x = np.concatenate([rng.uniform(-110, 88, 200000), rng.normal(0, 2, 200000)]).astype(np.float32)
    got = oracle.unary(x.view(np.uint32), 5).view(np.float32)
    want = np.exp(x.astype(np.float64)).astype(np.float32)
    assert int((got.view(np.uint32) != want.view(np.uint32)).sum()) == 0
    y = np.concatenate([rng.uniform(1, 5e8, 200000), 1 + rng.uniform(0, 4, 200000)]).astype(np.float32)
    got = oracle.unary(y.view(np.uint32), 6).view(np.float32)
    want = np.log(y.astype(np.float64)).astype(np.float32)
    assert int((got.view(np.uint32) != want.view(np.uint32)).sum()) == 0


def test_softplus_closed_form(oracle):
    v = np.float32([-30.0, -1.0, 0.0, 1.0, 19.5, 20.0, 20.5, 80.0])
    got = oracle.unary(v.view(np.uint32), 7).view(np.float32)
    e = np.exp(v.astype(np.float64)).astype(np.float32)
    want = np.where(v <= 20, np.log((e + np.float32(1)).astype(np.float64)).astype(np.float32), v)
    assert (got == want).all()
    assert got[-1] == 80.0 and got[-2] == 20.5    # identity above 20


# ------------------------------------------------------------- FP4 decode

def test_fp4_decode_closed_form_all_codes_all_scales(oracle):
    lev = np.float32([0, .5, 1, 1.5, 2, 3, 4, 6])
    scale_bytes = np.array([b for b in range(128) if b != 0x7F] + [0x80], np.uint8)
    rows = scale_bytes.size
    code_mat = np.tile(np.repeat(np.arange(16, dtype=np.uint8), 16), (rows, 1))
    zero = (scale_bytes & 0x7F) == 0
    code_mat[zero] = np.where(np.isin(code_mat[zero], (0, 8)), code_mat[zero], 0)
    packed = (code_mat[:, 0::2] | (code_mat[:, 1::2] << 4)).astype(np.uint8)
    sb = np.repeat(scale_bytes[:, None], 16, 1)
    blk = torch.from_numpy(sb).view(torch.float8_e4m3fn).float().numpy()
    for g in (1.0, 0.37, 2.0 ** -20):
        out, err = oracle.fp4_decode(16, packed, sb, g, rows, 256)
        assert err == 0
        c = code_mat.reshape(rows, 16, 16)
        val = lev[c & 7] * np.where(c & 8, np.float32(-1), np.float32(1))
        val = (val * blk[:, :, None]).astype(np.float32) * np.float32(g)
        want = val.astype(np.float32).astype(np.float16).view(np.uint16).reshape(rows, 256)
        assert (out == want).all()
    # code 8 decodes to -0.0 (0x8000) and code 0 to +0, except under the -0
    # block scale (byte 0x80), where IEEE sign rules flip both
    pos = scale_bytes < 0x80
    assert (out[pos, 16 * 8:16 * 9] == 0x8000).all() and (out[pos, :16] == 0).all()
    assert (out[~pos, 16 * 8:16 * 9] == 0).all() and (out[~pos, :16] == 0x8000).all()


def test_fp4_decode_error_bits(oracle):
    packed = np.full((1, 8), 0x11, np.uint8)
    out, err = oracle.fp4_decode(16, packed, np.uint8([[0x7F]]), 1.0, 1, 16)
    assert err & 1
    out, err = oracle.fp4_decode(16, packed, np.uint8([[0x00]]), 1.0, 1, 16)
    assert err & 4
    out, err = oracle.fp4_decode(16, packed, np.uint8([[0x40]]), 1e30, 1, 16)
    assert err & 8
    out, err = oracle.fp4_decode(16, packed, np.uint8([[0x40]]), 0.0, 1, 16)
    assert err & 32
    out, err = oracle.fp4_decode(16, packed, np.uint8([[0xC0]]), 1.0, 1, 16)
    assert err & 2
    out, err = oracle.fp4_decode(16, packed, np.uint8([[0x40]]), 1.0, 1, 14)
    assert err & 16


# ------------------------------------------------------ state-step invariants

def _ridge(oracle, layout, inp, sta, st):
    n8, n4, nz = cases.ridge_counts(layout)
    return oracle.state_step(oracle.MODE_RIDGE, n8, n4, nz, inp["x"], inp["dt"], inp["A"], inp["B"], inp["C"],
                             inp["D"], inp["dt_bias"], inp["perm"], sta["basis"], sta["lscale"], sta["pred"], st)


def test_zero_state_zero_input_stays_zero(oracle):
    rng = np.random.default_rng(3)
    for layout in cases.RIDGE_LAYOUTS:
        n8, n4, nz = cases.ridge_counts(layout)
        inp = cases.step_inputs(rng, 1, 3, 8, 16, 2)
        inp["x"][:] = 0
        st = cases.zero_packed_state(1, 8, 16, n8, n4, latent=True)
        y = _ridge(oracle, layout, inp, cases.ridge_statics(rng, 2, n8, n4, nz), st)
        assert not y.any()
        assert not st["lo"].any() and not st["hi"].any() and not st["q4"].any() and not st["latent"].any()
        # den floors at 1e-8, whose binary16 rounding underflows to 0
        assert not st["s8"].any() and not st["s4"].any()


def test_d_skip_passthrough(oracle):
    """B = C = 0, zero predictor: y = half(x * D) exactly and the carry only decays."""
    rng = np.random.default_rng(4)
    layout = "32_32_64"
    n8, n4, nz = cases.ridge_counts(layout)
    inp = cases.step_inputs(rng, 2, 1, 8, 16, 2)
    inp["B"][:] = 0
    inp["C"][:] = 0
    sta = cases.ridge_statics(rng, 2, n8, n4, nz)
    st = cases.random_packed_state(rng, 2, 8, 16, n8, n4, latent=True)
    y = _ridge(oracle, layout, inp, sta, st)
    x = cases.f16_to_f32(inp["x"])
    D = cases.f16_to_f32(inp["D"])
    want = (x * D[None, None, :, None]).astype(np.float32).astype(np.float16).view(np.uint16)
    assert (y == want).all()


def test_identity_step_is_idempotent(oracle):
    """A = 0 (decay 1) and B = 0: requantizing a dequantized row whose largest
    INT8 code is +-127 (and INT4 +-7) returns the same codes and scales."""
    rng = np.random.default_rng(5)
    for layout in cases.TIER_LAYOUTS:
        n8, n4, nz = cases.tier_counts(layout)
        inp = cases.step_inputs(rng, 1, 1, 8, 16, 2)
        inp["A"][:] = 0
        inp["B"][:] = 0
        st = cases.random_packed_state(rng, 1, 8, 16, n8, n4)
        # valid carries never hold -128: move such codes to -127 (lo nibble 0 -> 1)
        lo, hi = st["lo"], st["hi"]
        for sh in (0, 4):
            m = (((lo >> sh) & 15) == 0) & (((hi >> sh) & 15) == 8)
            lo[m] |= np.uint8(1 << sh)
        # force one +127 INT8 code and one -7 INT4 code per row (lane 0)
        st["lo"][..., 0] = (st["lo"][..., 0] & 0xF0) | 0xF
        st["hi"][..., 0] = (st["hi"][..., 0] & 0xF0) | 0x7
        q = st["q4"].copy()
        codes = np.stack((q & 15, q >> 4), -1).reshape(q.shape[:-1] + (n4,))
        codes = np.where(codes == 8, 9, codes)          # no -8 (outside +-7)
        codes[..., 0] = 9                               # -7
        st["q4"] = (codes[..., 0::2] | (codes[..., 1::2] << 4)).astype(np.uint8)
        # scales that are exact binary16 values representable as den*127 / den*7
        before = cases.copy_state(st)
        oracle.state_step(oracle.MODE_STORED, n8, n4, nz, inp["x"] * 0, inp["dt"], inp["A"], inp["B"], inp["C"],
                          inp["D"], inp["dt_bias"], inp["perm"], None, None, None, st)
        for k in ("lo", "hi", "q4", "s8", "s4"):
            assert (st[k] == before[k]).all(), (layout, k)


def test_multi_token_equals_sequential_single_tokens(oracle):
    rng = np.random.default_rng(6)
    layout = "24_48_56"
    n8, n4, nz = cases.ridge_counts(layout)
    inp = cases.step_inputs(rng, 2, 4, 8, 16, 2)
    sta = cases.ridge_statics(rng, 2, n8, n4, nz)
    st0 = cases.random_packed_state(rng, 2, 8, 16, n8, n4, latent=True)
    a = cases.copy_state(st0)
    y_all = _ridge(oracle, layout, inp, sta, a)
    b = cases.copy_state(st0)
    ys = []
    for t in range(4):
        one = {k: (np.ascontiguousarray(v[:, t:t + 1]) if k in ("x", "dt", "B", "C") else v) for k, v in inp.items()}
        ys.append(_ridge(oracle, layout, one, sta, b))
    assert all((a[k] == b[k]).all() for k in a)
    assert (np.concatenate(ys, 1) == y_all).all()


def test_ridge_reduces_to_tiers_without_latent_terms(oracle):
    """Zero basis, zero predictor and zero latent: the ridge row's INT8/INT4
    codes equal a tier step over the same carried lanes."""
    rng = np.random.default_rng(7)
    layout = "36_24_68"
    n8, n4, nz = cases.ridge_counts(layout)
    inp = cases.step_inputs(rng, 1, 2, 8, 16, 2)
    sta = dict(basis=np.zeros((2, nz, 2), np.uint16), lscale=cases.f16(np.full((2, 2), 1e-3)),
               pred=np.zeros((2, n8 + n4 + 2, nz), np.uint16))
    st = cases.random_packed_state(rng, 1, 8, 16, n8, n4, latent=True)
    st["latent"][:] = 0
    tier = {k: st[k].copy() for k in ("lo", "hi", "q4", "s8", "s4")}
    y_r = _ridge(oracle, layout, inp, sta, st)
    y_t = oracle.state_step(oracle.MODE_STORED, n8, n4, nz, inp["x"], inp["dt"], inp["A"], inp["B"], inp["C"],
                            inp["D"], inp["dt_bias"], inp["perm"], None, None, None, tier)
    for k in tier:
        assert (tier[k] == st[k]).all(), k
    assert not st["latent"].any()
    assert cases.rel_l2(cases.f16_to_f32(y_r), cases.f16_to_f32(y_t)) < 1e-3


def test_readout_matches_float64_restatement(oracle):
    """y against a float64 evaluation of the readout formula from the decoded
    pre-step carry (catches a dropped/transposed readout term)."""
    rng = np.random.default_rng(8)
    layout = "16_64_48"
    n8, n4, nz = cases.ridge_counts(layout)
    H, P, G = 8, 16, 2
    inp = cases.step_inputs(rng, 1, 1, H, P, G, dt_bias_zero=False)
    sta = cases.ridge_statics(rng, G, n8, n4, nz)
    st = cases.random_packed_state(rng, 1, H, P, n8, n4, latent=True)
    pre = cases.copy_state(st)
    y = cases.f16_to_f32(_ridge(oracle, layout, inp, sta, st))
    f = cases.f16_to_f32
    lo, hi, q4 = pre["lo"].astype(np.int32), pre["hi"].astype(np.int32), pre["q4"].astype(np.int32)
    l8 = np.stack((lo & 15, lo >> 4), -1).reshape(lo.shape[:-1] + (n8,))
    h8 = np.stack((hi & 15, hi >> 4), -1).reshape(hi.shape[:-1] + (n8,))
    q8 = ((h8 << 4) | l8).astype(np.int32); q8 -= 256 * (q8 > 127)
    n4c = np.stack((q4 & 15, q4 >> 4), -1).reshape(q4.shape[:-1] + (n4,)); n4c -= 16 * (n4c > 7)
    prior = np.concatenate([q8 * f(pre["s8"])[..., None], n4c * f(pre["s4"])[..., None]], -1).astype(np.float64)
    ls = f(sta["lscale"]).astype(np.float64)
    lat = torch.from_numpy(pre["latent"]).view(torch.float8_e4m3fn).double().numpy()
    for h in range(H):
        g = h // (H // G)
        perm = inp["perm"][g].astype(np.int64)
        bv = f(inp["B"][0, 0, g])[perm].astype(np.float64)
        cv = f(inp["C"][0, 0, g])[perm].astype(np.float64)
        dtv = math.log1p(math.exp(float(f(inp["dt"][0, 0, h])) + float(f(inp["dt_bias"])[h])))
        decay = math.exp(float(inp["A"][h]) * dtv)
        x = f(inp["x"][0, 0, h]).astype(np.float64)
        L8 = n8 + n4
        basis = f(sta["basis"][g]).astype(np.float64)
        pred = f(sta["pred"][g]).astype(np.float64)
        corr = pred @ cv[L8:]
        for p in range(P):
            z = lat[0, h, p] * ls[g]
            state = prior[0, h, p] * decay + bv[:L8] * dtv * x[p]
            out = state @ cv[:L8] + decay * (z @ (basis.T @ cv[L8:])) + x[p] * dtv * (bv[L8:] @ cv[L8:])
            out += x[p] * float(f(inp["D"])[h]) + decay * (prior[0, h, p] @ corr[:L8] + z @ corr[L8:])
            assert abs(y[0, 0, h, p] - out) <= 2e-3 * max(1.0, abs(out)), (h, p, y[0, 0, h, p], out)


# ---------------------------------------------------------------- s16 control

def _s16_inputs(rng, batch, L, H, P, G):
    inp = cases.step_inputs(rng, batch, L, H, P, G)
    st = cases.f16(rng.standard_normal((batch, H, P, 128)) * 0.5)
    return inp, st


def test_s16_unit_decay_zero_input_keeps_carry_and_reads_it_out(oracle):
    """A = 0 (decay exp(0) = 1), B = 0: the FP16 carry is unchanged and the
    readout is the float64 dot product with C plus x*D (closed form)."""
    rng = np.random.default_rng(71)
    inp, st = _s16_inputs(rng, 1, 2, 4, 32, 2)
    inp["A"][:] = 0
    inp["B"][:] = 0
    st0 = st.copy()
    y, _ = oracle.s16_step(inp["x"], inp["dt"], inp["A"], inp["B"], inp["C"], inp["D"], inp["dt_bias"], st)
    assert (st == st0).all()
    v = cases.f16_to_f32(st0).astype(np.float64)                       # [1,H,P,128]
    c = cases.f16_to_f32(inp["C"]).astype(np.float64)                  # [1,L,G,128]
    x = cases.f16_to_f32(inp["x"]).astype(np.float64)                  # [1,L,H,P]
    D = cases.f16_to_f32(inp["D"]).astype(np.float64)
    g = np.arange(4) // 2
    want = np.einsum("hpn,lhn->lhp", v[0], c[0][:, g]) + x[0] * D[None, :, None]
    got = cases.f16_to_f32(y[0]).astype(np.float64)
    assert np.allclose(got, want, rtol=2e-3, atol=2e-3)


def test_s16_input_lands_on_its_coordinate(oracle):
    """A = 0, B = e_j, x = 1: carry_j grows by exactly softplus(dt) (rounded
    to FP16), every other coordinate is untouched."""
    rng = np.random.default_rng(72)
    inp, st = _s16_inputs(rng, 1, 1, 2, 16, 1)
    inp["A"][:] = 0
    inp["B"][:] = 0
    j = 37
    inp["B"][0, 0, 0, j] = cases.f16(np.array([1.0]))[0]
    inp["x"][:] = cases.f16(np.array([1.0]))[0]
    st0 = cases.f16_to_f32(st.copy())
    oracle.s16_step(inp["x"], inp["dt"], inp["A"], inp["B"], inp["C"], inp["D"], inp["dt_bias"], st)
    after = cases.f16_to_f32(st)
    dt = cases.f16_to_f32(inp["dt"])[0, 0]                             # [H]
    sp = np.log1p(np.exp(dt.astype(np.float64))).astype(np.float32)
    want_j = (st0[..., j] + sp[None, :, None]).astype(np.float16).astype(np.float32)
    assert np.array_equal(after[..., j], want_j)
    mask = np.ones(128, bool)
    mask[j] = False
    assert np.array_equal(after[..., mask], st0[..., mask])


def test_s16_statistics_sum_stored_carry_per_tile(oracle):
    """Statistics = sum over tokens and the 16 rows of each P tile of
    |FP16 carry| after each token; ragged last tile."""
    rng = np.random.default_rng(73)
    inp, st = _s16_inputs(rng, 2, 3, 4, 40, 2)
    want = np.zeros((2, 4, 3, 128))
    cur = st.copy()
    for t in range(3):
        sl = slice(t, t + 1)
        oracle.s16_step(inp["x"][:, sl].copy(), inp["dt"][:, sl].copy(), inp["A"], inp["B"][:, sl].copy(),
                        inp["C"][:, sl].copy(), inp["D"], inp["dt_bias"], cur)
        a = np.abs(cases.f16_to_f32(cur).astype(np.float64))
        for tile in range(3):
            want[:, :, tile] += a[:, :, 16 * tile:16 * tile + 16].sum(2)
    st2 = st.copy()
    _, stats = oracle.s16_step(inp["x"], inp["dt"], inp["A"], inp["B"], inp["C"], inp["D"], inp["dt_bias"], st2,
                               collect_stats=True)
    assert (st2 == cur).all()                                           # one call == sequential calls
    assert np.allclose(stats, want, rtol=1e-6)


# ---------------------------------------------------------------- contracted update
# The reference kernels write the update as state * decay + (b * dt) * x and
# Triton fuses it into fma(state, decay, RN(RN(b * dt) * x)).  Each pin below
# builds one row whose first coordinate fixes the scale (b = 0 there, so both
# forms agree on it) and whose second coordinate is searched so that the
# fused and the separately rounded update give different stored values; the
# oracle must produce the fused one.  Expected values come from an exact
# rational evaluation of the fma.

from fractions import Fraction


def _rn32(fr):
    """Nearest binary32 to the rational `fr`, ties to even."""
    a = np.float32(float(fr))
    best = None
    for c in (np.nextafter(a, np.float32(-np.inf)), a, np.nextafter(a, np.float32(np.inf))):
        key = (abs(Fraction(float(c)) - fr), int(np.array(c, np.float32).view(np.uint32)) & 1)
        if best is None or key < best[0]:
            best = (key, np.float32(c))
    return best[1]


def _fma32(a, b, c):
    return _rn32(Fraction(float(a)) * Fraction(float(b)) + Fraction(float(c)))


def _round_half_away(q):
    q = np.asarray(q, np.float64)
    return np.sign(q) * np.floor(np.abs(q) + 0.5)


_DT, _A = 0.3, -0.7


def _dt_decay(oracle):
    dt = np.float32(np.float16(_DT))
    dtv = oracle.unary(np.array([dt], np.float32).view(np.uint32), 7).view(np.float32)[0]
    decay = oracle.unary(np.array([np.float32(_A) * dtv], np.float32).view(np.uint32), 5).view(np.float32)[0]
    return dtv, decay


def _search(priors, dtv, decay, code_of, valid=lambda u: np.ones(u.shape, bool), xs=(1.0,)):
    """(prior, b, x) whose fused and separately rounded updates give
    different codes (both updates `valid`); the first one verified exactly."""
    b = np.arange(0, 0x7C00, dtype=np.uint16)
    b = np.concatenate([b, b | 0x8000]).view(np.float16).astype(np.float32)
    bdt = (b * dtv).astype(np.float32)
    for x in xs:
        x = np.float32(np.float16(x))
        bx = (bdt * x).astype(np.float32)                       # RN(RN(b * dt) * x)
        for p in priors:
            p = np.float32(p)
            sep = (np.float32(p * decay) + bx).astype(np.float32)
            fus = (np.longdouble(p) * np.longdouble(decay) + bx.astype(np.longdouble)).astype(np.float32)
            cand = np.nonzero((code_of(fus) != code_of(sep)) & valid(fus) & valid(sep))[0]
            for i in cand[:4]:
                f = _fma32(p, decay, bx[i])
                if code_of(np.array([f]))[0] != code_of(sep[i:i + 1])[0]:
                    return p, np.float16(b[i]), x, f, sep[i]
    raise AssertionError("no discriminating pair found")


def _one_row_inputs(b_first, b_second, x=1.0, G=1):
    inp = dict(x=cases.f16(np.full((1, 1, 1, 1), x)), dt=cases.f16(np.full((1, 1, 1), _DT)),
               A=np.array([_A], np.float32), C=np.zeros((1, 1, G, 128), np.uint16),
               D=cases.f16(np.zeros(1)), dt_bias=cases.f16(np.zeros(1)),
               perm=np.arange(128, dtype=np.uint8)[None].repeat(G, 0))
    Bv = np.zeros(128, np.float32)
    Bv[0], Bv[1] = b_first, b_second
    inp["B"] = cases.f16(Bv[None, None, None])
    return inp


@pytest.mark.parametrize("mode", ["stored", "legacy"])
def test_tier_update_is_fused(oracle, mode):
    dtv, decay = _dt_decay(oracle)
    q0 = 113                                                  # coordinate 0 (b = 0) sets the maximum
    for s8 in (0.25, 0.3125, 0.375, 0.4375, 0.5625, 0.625):
        s8 = np.float32(s8)
        u0 = np.float32(np.float32(q0 * s8) * decay)
        den = max(np.float32(u0 / np.float32(127)), np.float32(1e-8))
        div = np.float32(np.float16(den)) if mode == "stored" else den

        def code_of(u):
            return np.clip(_round_half_away((u.astype(np.float32) / div).astype(np.float32)), -127, 127)
        try:   # coordinate 0 stays the maximum
            p, b, x, f, s = _search([q * s8 for q in range(-q0 + 20, q0 - 20) if q], dtv, decay, code_of,
                                    lambda u: np.abs(u) < u0)
            break
        except AssertionError:
            continue
    else:
        raise AssertionError("no discriminating pair found")
    q1 = int(round(float(p) / float(s8)))
    lo = np.zeros((1, 1, 1, 8), np.uint8)
    hi = np.zeros((1, 1, 1, 8), np.uint8)
    for n, q in ((0, q0), (1, q1)):
        byte = q & 0xFF
        lo[..., n // 2] |= np.uint8((byte & 15) << (4 * (n % 2)))
        hi[..., n // 2] |= np.uint8((byte >> 4) << (4 * (n % 2)))
    st = dict(lo=lo, hi=hi, q4=np.zeros((1, 1, 1, 32), np.uint8), s8=cases.f16(np.full((1, 1, 1), s8)),
              s4=cases.f16(np.zeros((1, 1, 1))))
    inp = _one_row_inputs(0.0, b, x)
    m = oracle.MODE_STORED if mode == "stored" else oracle.MODE_LEGACY
    oracle.state_step(m, 16, 64, 48, inp["x"], inp["dt"], inp["A"], inp["B"], inp["C"], inp["D"], inp["dt_bias"],
                      inp["perm"], None, None, None, st)
    byte = ((int(st["hi"][0, 0, 0, 0]) >> 4) << 4) | (int(st["lo"][0, 0, 0, 0]) >> 4)
    got = byte - 256 * (byte > 127)
    assert got == code_of(np.array([f]))[0] != code_of(np.array([s]))[0]


def test_dense3_update_is_fused(oracle):
    """Observed through the readout: with C = e_1 and D = 0, y = half(u_1)."""
    dtv, decay = _dt_decay(oracle)
    sc = np.float32(0.25)

    def code_of(u):
        return u.astype(np.float32).astype(np.float16).view(np.uint16).astype(np.int64)

    p, b, x, f, s = _search([q * sc for q in (-4, -3, -2, -1, 1, 2, 3)], dtv, decay, code_of)
    q = np.zeros(128, np.int64)
    q[1] = int(round(float(p) / float(sc)))
    codes = np.zeros((1, 1, 1, 3, 16), np.uint8)
    for k in range(3):
        for j in range(16):
            codes[0, 0, 0, k, j] = sum((((q[8 * j + bit] & 7) >> k) & 1) << bit for bit in range(8))
    st = dict(codes=codes, scales=cases.f16(np.full((1, 1, 1, 2), sc)))
    inp = _one_row_inputs(0.0, b, x)
    inp["C"][0, 0, 0, 1] = cases.f16(np.array([1.0]))[0]
    y = oracle.dense3_step(0, inp["x"], inp["dt"], inp["A"], inp["B"], inp["C"], inp["D"], inp["dt_bias"],
                           inp["perm"], st)
    assert int(y[0, 0, 0, 0]) == code_of(np.array([f]))[0] != code_of(np.array([s]))[0]


def test_s16_update_is_fused(oracle):
    dtv, decay = _dt_decay(oracle)

    def code_of(u):
        return u.astype(np.float32).astype(np.float16).view(np.uint16).astype(np.int64)

    vals = np.arange(0x3800, 0x4000, 7, dtype=np.uint16).view(np.float16).astype(np.float32)
    p, b, x, f, s = _search(vals, dtv, decay, code_of)
    st = np.zeros((1, 1, 1, 128), np.uint16)
    st[0, 0, 0, 1] = cases.f16(np.array([p]))[0]
    inp = _one_row_inputs(0.0, b, x)
    oracle.s16_step(inp["x"], inp["dt"], inp["A"], inp["B"], inp["C"], inp["D"], inp["dt_bias"], st)
    assert int(st[0, 0, 0, 1]) == code_of(np.array([f]))[0] != code_of(np.array([s]))[0]


def test_encode_legacy_matches_reference_vectors(oracle):
    """The oracle's legacy diagnostic encoder (state_codec.py:299-331) against
    the reference's own encode_state_ outputs (tests/golden/encode_legacy_vectors.npz,
    written by tests/golden/make_encode_legacy_vectors.py): every nibble
    plane byte and stored scale bit-exact, over Gaussian rows, exact
    half-integer codes and one ulp either side (sign(z)*floor(|z|+0.5) rounds
    ties away from zero, so a round-half-even encoder fails here), the 1e-8
    scale floor, zero and signed-zero rows."""
    g = np.load(Path(__file__).resolve().parent / "golden" / "encode_legacy_vectors.npz")
    got = oracle.encode_legacy(g["dense"])
    for k in ("lo", "hi", "q4", "s8", "s4"):
        assert np.array_equal(got[k], g[k]), k
    # the tie rows do exercise half-away rounding: an encoder rounding ties to
    # even gives different codes on them
    dense = g["dense"].reshape(-1, 128)
    ties = dense[96:160:3, 1:16]
    assert np.any(np.abs(ties - np.trunc(ties)) == 0.5)
    assert not np.array_equal(np.rint(ties), np.sign(ties) * np.floor(np.abs(ties) + 0.5))
