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


# residual bounds of the magic-number quantizer's residual form (the form
# the device used before its two-sided form, below; the identity both rest on)
RESIDUAL_OK8 = 0.5 - 2.0 ** -16
RESIDUAL_OK4 = 0.5 - 2.0 ** -19


def test_residual_rounding_quantizer_equals_roundf_of_ieee_division(oracle):
    """The magic-number quantizer in its residual form keeps rint(v * RN(1/d))
    (the low byte of fma(v, y, 1.5 2^23 + bias)) whenever the rounding residual
    |f| is within the bound, and recomputes the rest exactly: every kept code
    equals roundf(v / d) and its byte is code + bias, for lim 127, 7 and 3,
    random quotients and every half-integer boundary +-40 ulps.  The near-tie
    cases do reach the exact path."""
    bad, flagged = oracle.check_residual_round(20261202, 20_000_000, 400_000, RESIDUAL_OK8, RESIDUAL_OK4)
    assert bad == 0
    assert flagged > 400_000   # boundary cases within the margin went to the exact path


def test_residual_rounding_without_margin_is_caught(oracle):
    """Planted mistake: keeping every magic-number code (no residual margin,
    ties to even instead of away from zero) disagrees with roundf(v / d) on
    the boundary cases, so the check above has teeth."""
    bad, _ = oracle.check_residual_round(20261202, 0, 20_000, 0.5, 0.5)
    assert bad > 0


# relative offset of the two-sided quantizer's reciprocals (m2r_device.h)
TWO_SIDED_REL = 2.0 ** -22


def test_two_sided_rounding_quantizer_equals_roundf_of_ieee_division(oracle):
    """The device's unclamped quantizer in its two-sided form: the codes of
    fma(v, y_hi, magic) and fma(v, y_lo, magic), with y = RN(1/d) and y_hi/lo
    = RN(y (1 +- 2^-22)), are kept when they agree, and every kept code must
    equal roundf(v / d) with its byte code + bias (lim 127, 7 and 3, random
    quotients and every half-integer boundary +-40 ulps).  Near-ties reach
    the exact path; so do fewer random cases than with a residual bound of
    the same width would reach by chance."""
    bad, flagged = oracle.check_two_sided_round(20261203, 20_000_000, 400_000, TWO_SIDED_REL)
    assert bad == 0
    assert flagged > 400_000   # boundary cases within the window went to the exact path


@pytest.mark.parametrize("rel", [0.0, 2.0 ** -25])
def test_two_sided_rounding_without_enough_margin_is_caught(oracle, rel):
    """Planted mistakes: no offset (one code kept always, ties to even) and
    an offset below the reciprocal's own rounding error both keep codes that
    disagree with roundf(v / d) on the boundary cases."""
    bad, _ = oracle.check_two_sided_round(20261203, 0, 20_000, rel)
    assert bad > 0


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


# --------------------------------------------- latent update and its E4M3 bytes

def _e4m3_byte(q):
    """float32 -> E4M3FN byte by torch's conversion (round to nearest even)."""
    return int(torch.tensor([float(q)], dtype=torch.float32).to(torch.float8_e4m3fn).view(torch.uint8)[0])


def _e4m3_value(byte):
    return float(torch.tensor([byte], dtype=torch.uint8).view(torch.float8_e4m3fn).float()[0])


def _latent_expect(z, decay, xdt, dot_b, ls):
    """Exact rational restatement of one latent step
    (scripts/fp4_zero_predictor_codec_v1.py:149-152): z' = RN(z*decay + RN(xdt*dot_b)),
    byte = E4M3(clamp(RN(z'/ls), -448, 448)).  Returns (z', byte)."""
    inp = _rn32(Fraction(float(xdt)) * Fraction(float(dot_b)))
    zn = _rn32(Fraction(float(z)) * Fraction(float(decay)) + Fraction(float(inp)))
    q = _rn32(Fraction(float(zn)) / Fraction(float(ls)))
    return zn, _e4m3_byte(min(max(float(q), -448.0), 448.0))


def _one_hot_latent_call(oracle, layout, x0, lat0, *, dt, A, b, c, ls, d0, d1, L2=True):
    """One head of P rows through the ridge oracle with a one-hot dead-tier
    basis (e0 = 0.5 at dead lane d0, e1 = 0.5 at d1), B and C nonzero only at
    d0/d1 (token 0), zero predictor, zero carried tiers, D = 0.  With L2 a
    second token follows with x = 0, B = 0 and C = 2 at d0: its readout is
    exactly half(decay * z0) of the requantized latent coefficient."""
    n8, n4, nz = cases.ridge_counts(layout)
    rows = len(x0)
    L = 2 if L2 else 1
    live = n8 + n4
    x = np.zeros((1, L, 1, rows), np.float32)
    x[0, 0, 0] = x0
    Bm = np.zeros((1, L, 1, 128), np.float32)
    Cm = np.zeros((1, L, 1, 128), np.float32)
    Bm[0, 0, 0, live + d0], Bm[0, 0, 0, live + d1] = b
    Cm[0, 0, 0, live + d0], Cm[0, 0, 0, live + d1] = c
    if L2:
        Cm[0, 1, 0, live + d0] = 2.0
    inp = dict(x=cases.f16(x), dt=cases.f16(np.full((1, L, 1), dt)), A=np.array([A], np.float32),
               B=cases.f16(Bm), C=cases.f16(Cm), D=cases.f16(np.zeros(1)), dt_bias=cases.f16(np.zeros(1)),
               perm=np.arange(128, dtype=np.uint8)[None])
    basis = np.zeros((1, nz, 2), np.float32)
    basis[0, d0, 0] = 0.5
    basis[0, d1, 1] = 0.5
    sta = dict(basis=cases.f16(basis), lscale=cases.f16(np.array([ls], np.float32)),
               pred=np.zeros((1, n8 + n4 + 2, nz), np.uint16))
    st = cases.zero_packed_state(1, 1, rows, n8, n4, latent=True)
    st["latent"][0, 0] = np.asarray(lat0, np.uint8)
    y = _ridge(oracle, layout, inp, sta, st)
    return st["latent"][0, 0], y


def _latent_case_table():
    """(x, initial byte of coefficient 0) rows for ls0 = 1/16, dt = 32
    (softplus identity branch), decay 1, b0 = 1/16: 16 z0' = v0 + 16 x exactly,
    so these hit E4M3 ties (to even), the +-448 clamp, the subnormal range and
    signed zero."""
    one, v256, mv256 = 0x38, 0x78, 0xF8
    return [
        (2.0 ** -8, one),            # 1.0625: tie 1.0 | 1.125 -> 1.0 (even)
        (3 * 2.0 ** -8, one),        # 1.1875: tie 1.125 | 1.25 -> 1.25
        (5 * 2.0 ** -8, one),        # 1.3125: tie 1.25 | 1.375 -> 1.25
        (2.0 ** -7, one),            # 1.125 exact
        (1.0, v256),                 # 272: tie 256 | 288 -> 256
        (3.0, v256),                 # 304: tie 288 | 320 -> 320
        (12.0, v256),                # 448 exact
        (13.0, v256),                # 464 -> clamp 448
        (46.5, v256),                # 1000 -> clamp 448
        (-20.0, mv256),              # -576 -> clamp -448
        (-12.0, mv256),              # -448 exact
        (3 * 2.0 ** -14, 0x00),      # 1.5 * 2^-9: tie 2^-9 | 2^-8 -> 2^-8 (even)
        (2.0 ** -14, 0x00),          # 2^-10: tie 0 | 2^-9 -> 0 (even)
        (2.0 ** -14 + 2.0 ** -24, 0x00),   # just above: 2^-9
        (-(2.0 ** -14), 0x00),       # -2^-10: tie -> -0
        (-0.0, 0x80),                # -0 stays -0
        (0.0, 0x00),
        (-2.0 ** -8, 0xB8),          # -1.0625: tie -> -1.0
    ]


def test_latent_update_known_answers(oracle):
    """The ridge latent step and its E4M3 requantization
    (scripts/fp4_zero_predictor_codec_v1.py:149-152, 176-179) on a one-hot basis,
    against exact rational arithmetic and torch's E4M3FN conversion: E4M3
    ties to even, the +-448 clamp, subnormals, signed zero; coefficient 1
    through a non-power-of-two latent scale; and the second token's readout,
    which must use the requantized coefficient."""
    layout = "32_32_64"
    d0, d1 = 3, 66
    b = (2.0 ** -4, 2.0 ** -3)               # b0 != b1: a swapped e0/e1 changes every row
    c = (0.75, -1.5)                          # C differs from B at both dead lanes
    # coefficient 1's scale: binary16 0x1468, for which z1' = 1.9375 ls1 (an
    # E4M3 tie, to even 2.0) is reached from 1.875 ls1 with x = ls1/32, while
    # z1' * RN(1/ls1) rounds to 1.875: a quotient by the rounded reciprocal fails
    ls1 = float(np.uint16(0x1468).view(np.float16))
    ls = (2.0 ** -4, ls1)
    table = _latent_case_table()
    special1 = {len(table): 0x3F, len(table) + 1: 0xBF}
    table += [(ls1 / 32, 0x38), (-ls1 / 32, 0x38)]
    rng = np.random.default_rng(151)
    while len(table) < 64:                    # plus random rows
        table.append((float(np.float16(rng.normal(0, 4))), int(cases.random_e4m3_bytes(rng, (1,))[0])))
    x0 = np.array([t[0] for t in table], np.float32)
    lat0 = np.stack([np.array([t[1] for t in table], np.uint8),
                     cases.random_e4m3_bytes(rng, (len(table),))], -1)
    for r, byte in special1.items():
        lat0[r, 1] = byte
    got, y = _one_hot_latent_call(oracle, layout, x0, lat0, dt=32.0, A=0.0, b=b, c=c, ls=ls, d0=d0, d1=d1)
    dtv, decay = np.float32(32.0), np.float32(1.0)
    swapped_differs = False
    for r, (xv, _) in enumerate(table):
        xdt = np.float32(np.float32(np.float16(xv)) * dtv)
        for k in range(2):
            z = np.float32(_e4m3_value(int(lat0[r, k])) * np.float32(np.float16(ls[k])))
            zn, byte = _latent_expect(z, decay, xdt, np.float32(0.5 * b[k]), np.float16(ls[k]))
            # token 1 (x = 0, B = 0): z'' = RN(zq + 0), so -0 becomes +0
            zq = np.float32(np.float32(_e4m3_value(byte)) * np.float32(np.float16(ls[k])))
            _, byte = _latent_expect(zq, decay, np.float32(0.0), np.float32(0.0), np.float16(ls[k]))
            assert int(got[r, k]) == byte, (r, k, xv, float(zn), hex(int(got[r, k])), hex(byte))
            _, wrong = _latent_expect(z, decay, xdt, np.float32(0.5 * b[1 - k]), np.float16(ls[k]))
            swapped_differs |= wrong != byte
        # token 1: y = half(z0 requantized), not half(z0')
        zq = np.float32(_e4m3_value(int(got[r, 0])) * np.float32(2.0 ** -4))
        assert int(y[0, 1, 0, r]) == int(cases.f16(np.array([zq]))[0]), r
    assert swapped_differs
    assert [int(got[r, 1]) for r in special1] == [0x40, 0xC0]
    # the table's first rows are ties whose requantized value differs from z'
    z0n = (np.float32(1.0) + x0[:2]).astype(np.float32) / 16
    assert not np.array_equal(cases.f16(z0n), y[0, 1, 0, :2])


def test_latent_update_general_decay_matches_exact_arithmetic(oracle):
    """Random x, dt (softplus branch), A (decay < 1), B at the dead lanes,
    initial latent bytes and latent scales: every byte equals the exact
    rational z' = RN(z*decay + RN(RN(x*dt)*dot_b)) requantized, with dt and
    decay from the oracle's exp/log (pinned against libm above)."""
    layout = "44_8_76"
    d0, d1 = 0, 79
    rng = np.random.default_rng(152)
    for trial in range(6):
        dt = float(np.float16(rng.normal(0, 1)))
        A = float(-np.exp(rng.uniform(0, np.log(16))))
        b = tuple(float(np.float16(v)) for v in rng.normal(0, 1, 2))
        c = tuple(float(np.float16(v)) for v in rng.normal(0, 1, 2))
        ls = tuple(float(np.float16(v)) for v in np.exp(rng.normal(-6, 1, 2)))
        x0 = cases.f16_to_f32(cases.f16(rng.normal(0, 2, 64)))
        lat0 = cases.random_e4m3_bytes(rng, (64, 2))
        got, _ = _one_hot_latent_call(oracle, layout, x0, lat0, dt=dt, A=A, b=b, c=c, ls=ls, d0=d0, d1=d1,
                                      L2=False)
        dtv = oracle.unary(np.array([np.float32(np.float16(dt))]).view(np.uint32), 7).view(np.float32)[0]
        decay = oracle.unary(np.array([np.float32(A) * dtv], np.float32).view(np.uint32), 5).view(np.float32)[0]
        for r in range(64):
            xdt = np.float32(x0[r] * dtv)
            for k in range(2):
                dot_b = np.float32(np.float32(0.5) * np.float32(np.float16(b[k])))
                z = np.float32(np.float32(_e4m3_value(int(lat0[r, k]))) * np.float32(np.float16(ls[k])))
                _, byte = _latent_expect(z, decay, xdt, dot_b, np.float16(ls[k]))
                assert int(got[r, k]) == byte, (trial, r, k)


# -------------------------------------- dense 3-bit requantization and bit planes

def _d3_expect(u, half_scale_policy="den"):
    """state_codec_dense3.py:133-145 for one row of 128 updated values u
    (float32), by exact rationals: den = max(RN(amax/3), 1e-8) per half,
    q = clamp(roundf(RN(u/den)), +-3) (ties away from zero), stored half(den).
    half_scale_policy="stored" divides by the stored binary16 scale instead
    (a plausible mistake the pin must reject)."""
    q = np.zeros(128, np.int64)
    scales = np.zeros(2, np.uint16)
    for hh in range(2):
        seg = u[64 * hh:64 * hh + 64]
        amax = max(abs(Fraction(float(v))) for v in seg)
        den = max(_rn32(amax / 3), np.float32(1e-8))
        st = np.float16(den)
        div = Fraction(float(den)) if half_scale_policy == "den" else Fraction(float(st))
        for i, v in enumerate(seg):
            if div == 0:
                qq = 0
            else:
                t = Fraction(float(_rn32(Fraction(float(v)) / div)))
                mag = math.floor(abs(t) + Fraction(1, 2))
                qq = int(mag if t >= 0 else -mag)
            q[64 * hh + i] = min(max(qq, -3), 3)
        scales[hh] = st.view(np.uint16)
    return q, scales


def _d3_planes(q):
    """Bit planes of 3-bit two's-complement codes, by numpy's little-endian
    bit packing (coordinate 8j + b is bit b of byte j of each plane)."""
    u = (np.asarray(q, np.int64) & 7).astype(np.uint8)
    return np.stack([np.packbits(((u >> k) & 1).astype(np.uint8), bitorder="little") for k in range(3)])


def _d3_call(oracle, prior_q, prior_s, x, bvec):
    """One head of P rows through the dense 3-bit oracle with decay 1 (A = 0)
    and dt = 32 (softplus's identity branch): u = RN(prior + RN(32 b x)) per
    coordinate, exactly known.  Returns (state after, u per row)."""
    P = len(x)
    codes = np.stack([_d3_planes(q).reshape(48) for q in prior_q]).reshape(1, 1, P, 3, 16)
    scales = cases.f16(prior_s).reshape(1, 1, P, 2)
    B = np.zeros((1, 1, 1, 128), np.float32)
    B[0, 0, 0] = bvec
    inp = dict(x=cases.f16(np.asarray(x, np.float32).reshape(1, 1, 1, P)), dt=cases.f16(np.full((1, 1, 1), 32.0)),
               A=np.zeros(1, np.float32), B=cases.f16(B), C=cases.f16(np.zeros((1, 1, 1, 128))),
               D=cases.f16(np.zeros(1)), dt_bias=cases.f16(np.zeros(1)))
    st = dict(codes=codes, scales=scales.copy())
    oracle.dense3_step(0, inp["x"], inp["dt"], inp["A"], inp["B"], inp["C"], inp["D"], inp["dt_bias"],
                       np.arange(128, dtype=np.uint8)[None], st)
    f = lambda a: Fraction(float(a))
    bdt = (cases.f16_to_f32(inp["B"][0, 0, 0]) * np.float32(32.0)).astype(np.float32)
    us = []
    for r in range(P):
        prior = (np.asarray(prior_q[r]) * np.repeat(cases.f16_to_f32(scales[0, 0, r]), 64)).astype(np.float32)
        xv = cases.f16_to_f32(inp["x"][0, 0, 0, r])
        us.append(np.array([_rn32(f(prior[n]) + f(np.float32(bdt[n] * xv))) for n in range(128)], np.float32))
    return st, us


def test_dense3_requantization_and_packing_known_answers(oracle):
    """The dense 3-bit requantization and bit-plane packing
    (mamba2_recall/state_codec_dense3.py:133-145) with decay 1 and a known
    input term (u = RN(prior + RN(32 b x)) exactly): codes, planes and stored
    scales against exact rationals, numpy's little-endian bit packing and
    numpy's binary16 rounding.  Rows cover exact k + 1/2 quotients (ties away
    from zero: a round-half-even quantizer fails), the 1e-8 denominator floor
    (binary16 scale 0), and random rows on which dividing by the stored
    binary16 scale instead of den gives other codes."""
    rng = np.random.default_rng(133)
    # call 1: exact ties.  Coordinates 0 and 64 carry 3 * 2^m (code 3, scale
    # 2^m), so den = 2^m in both halves; every other coordinate gets only the
    # input term (k + 1/2) 2^m: b_n = (k + 1/2) 2^m0 / 32, x_r = 2^(m_r - m0)
    m0, P = -4, 8
    halves = np.resize(np.array([0.5, -0.5, 1.5, -1.5, 2.5, -2.5]), 128)
    halves[0] = halves[64] = 0.0
    bvec = (halves * 2.0 ** m0 / 32).astype(np.float32)
    prior_q = np.zeros((P, 128), np.int64)
    prior_q[:, 0] = prior_q[:, 64] = 3
    ms = np.arange(P) - 6
    prior_s = np.repeat((2.0 ** ms)[:, None], 2, 1).astype(np.float32)
    st, us = _d3_call(oracle, prior_q, prior_s, 2.0 ** (ms - m0), bvec)
    for r in range(P):
        q, sc = _d3_expect(us[r])
        assert np.array_equal(us[r] / np.float32(2.0 ** ms[r]), halves + 3 * (np.arange(128) % 64 == 0))
        assert np.array_equal(st["codes"][0, 0, r], _d3_planes(q)), r
        assert np.array_equal(st["scales"][0, 0, r], sc), r
        h = halves[1:64]                                                  # ties away from zero
        assert (q[1:64] == np.sign(h) * np.floor(np.abs(h) + 0.5)).all()
        assert (q[1:64] != np.rint(h)).any()
    # call 2: zero priors and input terms below 3e-8 (rows 0-3, x = 2^-24: den
    # is the 1e-8 floor, stored scale 0), then random priors and input terms
    P = 40
    prior_q = rng.integers(-4, 4, (P, 128))
    prior_q[:4] = 0
    prior_s = np.exp(rng.normal(-3, 0.5, (P, 2))).astype(np.float16).astype(np.float32)
    x = cases.f16_to_f32(cases.f16(rng.normal(0, 1, P)))
    x[:4] = 2.0 ** -24
    bvec = cases.f16_to_f32(cases.f16(rng.normal(0, 0.004, 128)))
    st, us = _d3_call(oracle, prior_q, prior_s, x, bvec)
    stored_differs = 0
    for r in range(P):
        q, sc = _d3_expect(us[r])
        assert np.array_equal(st["codes"][0, 0, r], _d3_planes(q)), r
        assert np.array_equal(st["scales"][0, 0, r], sc), r
        stored_differs += int(not np.array_equal(q, _d3_expect(us[r], "stored")[0]))
    assert not st["scales"][0, 0, :4].any() and st["codes"][0, 0, :4].any()
    assert stored_differs > 0           # dividing by half(den) would be caught


# ------------------------------------------------------------- G64 closed form

def test_fp4_g64_closed_form_all_codes_scale_sweep(oracle):
    """G64 decode (mamba2_recall/fp4.py:151-154, G64 branch): w =
    half(lev[c & 7] * sign(c) * float(f16 scale)) with one rounding and no
    global scale, for all 16 codes x every non-negative finite binary16 scale
    (subnormals, +-0, 65504), against numpy's IEEE float32 product and
    binary16 rounding; products that overflow binary16 raise only the
    nonfinite-weight bit.  A global scale passed with G64 is ignored."""
    lev = np.float32([0, .5, 1, 1.5, 2, 3, 4, 6])
    scale_bits = np.concatenate([np.arange(0, 0x7C00, dtype=np.uint16), np.uint16([0x8000])])
    rows = scale_bits.size
    codes = np.tile(np.repeat(np.arange(16, dtype=np.uint8), 4), (rows, 1))   # 64 columns
    zero = (scale_bits & 0x7FFF) == 0
    codes[zero] = np.where(np.isin(codes[zero], (0, 8)), codes[zero], 0)
    packed = (codes[:, 0::2] | (codes[:, 1::2] << 4)).astype(np.uint8)
    sc = scale_bits[:, None].copy()
    val = lev[codes & 7] * np.where(codes & 8, np.float32(-1), np.float32(1))
    with np.errstate(over="ignore"):
        want = (val * sc.view(np.float16).astype(np.float32)).astype(np.float32).astype(np.float16).view(np.uint16)
    overflow = ((want & 0x7FFF) >= 0x7C00).any()
    assert overflow
    for g in (1.0, 0.37):
        out, err = oracle.fp4_decode(64, packed, sc, g, rows, 64)
        assert err == 8, err
        assert np.array_equal(out, want)
    ok = (scale_bits & 0x7FFF) < 0x5400           # |6 * scale| < 65504: no overflow
    out, err = oracle.fp4_decode(64, np.ascontiguousarray(packed[ok]), np.ascontiguousarray(sc[ok]), 3.0,
                                 int(ok.sum()), 64)
    assert err == 0 and np.array_equal(out, want[ok])
    # the global scale must not apply, and the scale is binary16, not E4M3
    with np.errstate(over="ignore"):
        scaled = (val * sc.view(np.float16).astype(np.float32) * np.float32(0.37)).astype(np.float16).view(np.uint16)
    assert not np.array_equal(scaled, want)
    # signs of zero: code 8 under a +0 scale is -0, code 0 under -0 is -0
    assert (out[0, 32:36] == 0x8000).all() and (out[0, :4] == 0).all()
    neg0 = np.nonzero(scale_bits == 0x8000)[0][0]
    full, _ = oracle.fp4_decode(64, packed, sc, 1.0, rows, 64)
    assert (full[neg0, :4] == 0x8000).all() and (full[neg0, 32:36] == 0).all()


def test_latent_update_is_fused(oracle):
    """The latent step is one fused multiply-add, z' = fma(z, decay,
    RN(RN(x*dt)*dot_b)), like the tier update: a row whose fused and
    separately rounded z' give different E4M3 bytes (found by search, checked
    with exact rationals) must store the fused one."""
    dtv, decay = _dt_decay(oracle)
    ls = np.float16(2.0 ** -6)
    b = np.arange(0, 0x7C00, dtype=np.uint16)
    b = np.concatenate([b, b | 0x8000]).view(np.float16).astype(np.float32)
    dot_b = (np.float32(0.5) * b).astype(np.float32)
    x = np.float32(1.0)
    inp = (np.float32(x * dtv) * dot_b).astype(np.float32)             # RN(RN(x*dt)*dot_b)

    def byte_of(u):
        q = np.clip((u.astype(np.float32) / np.float32(ls)).astype(np.float32), -448, 448)
        return torch.from_numpy(q.astype(np.float32)).to(torch.float8_e4m3fn).view(torch.uint8).numpy()

    found = None
    for vb in range(0x08, 0x78):
        z = np.float32(np.float32(_e4m3_value(vb)) * np.float32(ls))
        sep = (np.float32(z * decay) + inp).astype(np.float32)
        fus = (np.longdouble(z) * np.longdouble(decay) + inp.astype(np.longdouble)).astype(np.float32)
        for i in np.nonzero(byte_of(fus) != byte_of(sep))[0][:4]:
            f = _fma32(z, decay, inp[i])
            if byte_of(np.array([f]))[0] != byte_of(sep[i:i + 1])[0]:
                found = (vb, float(b[i]), f, sep[i])
                break
        if found:
            break
    assert found, "no discriminating row found"
    vb, bv, f, s = found
    # dead lane 0 carries e0 = 0.5 and B = bv; dt and A as in the search
    got, _ = _one_hot_latent_call(oracle, "32_32_64", np.float32([x]), np.uint8([[vb, 0]]), dt=_DT, A=_A,
                                  b=(bv, 0.0), c=(0.0, 0.0), ls=(float(ls), 1.0), d0=0, d1=1, L2=False)
    assert int(got[0, 0]) == int(byte_of(np.array([f]))[0]) != int(byte_of(np.array([s]))[0])


# ------------------------------------------------- PyTorch-CPU restatements

def test_torch_cpu_decode_rows_matches_reference_vectors():
    """oracle/torch_cpu.decode_rows against the reference decode_state's own
    outputs in packed lane order (sq3p25 16/64/48; arbitrary bytes, zero,
    negative-zero, subnormal and negative scales), bit for bit."""
    from pathlib import Path
    from oracle import torch_cpu
    g = np.load(Path(__file__).resolve().parent / "golden" / "decode_state_vectors.npz")
    t = {k: torch.from_numpy(g[f"sq_{k}"]) for k in ("lo", "hi", "q4", "s8", "s4")}
    out = torch_cpu.decode_rows(t["lo"], t["hi"], t["q4"], t["s8"].view(torch.int16), t["s4"].view(torch.int16), 16, 64)
    assert np.array_equal(out.numpy().view(np.uint32), g["sq_decode"].view(np.uint32))


def test_torch_cpu_fp4_decode_matches_c_oracle(oracle):
    """oracle/torch_cpu.fp4_g16_decode against the C oracle's G16 decode: all
    16 codes in every non-NaN block byte (signs included) and random rows,
    under three global scales, bit for bit."""
    from oracle import torch_cpu
    rng = np.random.default_rng(9)
    # every finite non-negative block byte; a zero block (0x00, 0x80) may
    # only hold the zero codes 0 and 8 (fp4.py:247), which its row then repeats
    blocks = np.array([b for b in range(256) if (b & 0x7F) != 0x7F and not (b & 0x80 and b != 0x80)], np.uint8)
    rows = len(blocks)
    codes = np.tile(np.arange(16, dtype=np.uint8), (rows, 1))          # one group per row, all codes
    codes[(blocks & 0x7F) == 0] = np.tile(np.array([0, 8], np.uint8), 8)
    packed = (codes[:, 0::2] | (codes[:, 1::2] << 4)).astype(np.uint8)
    packed = np.concatenate([packed, rng.integers(0, 256, (rows, 56), dtype=np.uint16).astype(np.uint8)], axis=1)
    nonzero = blocks[(blocks & 0x7F) != 0]
    sb = np.stack([blocks] + [rng.choice(nonzero, rows) for _ in range(7)], axis=1).astype(np.uint8)
    for g in (np.float32(1.0), np.float32(0.0123), np.float32(3.1e-5)):
        want, err = oracle.fp4_decode(16, packed, sb, g, rows, 128)
        assert err == 0
        got = torch_cpu.fp4_g16_decode(torch.from_numpy(packed), torch.from_numpy(sb), float(g))
        assert np.array_equal(got.numpy().view(np.uint16), want)


def test_s16_statistics_fixed_summation_order(oracle):
    """The s16 calibration statistics are binary32 sums in one fixed order:
    each row over the tokens in order, a 4-row sub-tile as (r0 + r1) + (r2 +
    r3), the four sub-tiles of a 16-row tile as ((T0 + T1) + T2) + T3
    (state_codec.py:100-102 per program, :255-261 on the host).  With x = 0
    and decay exactly 1 (A = -1e-30) the FP16 carry is the state itself, so
    the rows can be chosen where the plausible other orders round
    differently: 131008 + 2^-8 is a tie that rounds back to 131008 (even
    significand), while 131008 + 2^-7 is exact.  Sequential row sums, or a
    pairwise fold of the sub-tiles, give 131008 where the fixed order gives
    131008 + 2^-7; a float64 accumulation gives 131008 + 2^-7 + 2^-8 in the
    second case."""
    H, P, G, L = 1, 32, 1, 2
    big, small = 65504.0, 2.0 ** -8
    state = np.zeros((1, H, P, 128), np.float32)
    # tile 0 (rows 0-15): sub-tile 0 holds big, big, small, small -> (2 big) + 2^-7
    state[0, 0, 0:2, 0] = big
    state[0, 0, 2:4, 0] = small
    # tile 1 (rows 16-31): sub-tiles 2^-8... T0 = 2 big, T1 = 0, T2 = T3 = small
    state[0, 0, 16:18, 1] = big
    state[0, 0, 24, 1] = small
    state[0, 0, 28, 1] = small
    # coordinate 2: two tokens of the same rows sum per row first (token order)
    state[0, 0, 5, 2] = 3.0
    st = cases.f16(state)
    x = np.zeros((1, L, H, P), np.uint16)
    dt = cases.f16(np.zeros((1, L, H)))
    A = np.full(H, -1e-30, np.float32)
    B = cases.f16(np.ones((1, L, G, 128)))
    C = cases.f16(np.ones((1, L, G, 128)))
    D = cases.f16(np.zeros(H))
    db = cases.f16(np.zeros(H))
    carry = st.copy()
    _, stats = oracle.s16_step(x, dt, A, B, C, D, db, carry, collect_stats=True)
    assert np.array_equal(carry, st), "decay 1 and x = 0 must leave the carry unchanged"
    f = np.float32
    two_big = f(big) + f(big)
    # per token: tile 0 coordinate 0 is 2 big + 2^-7 exactly; over two tokens
    # each row is summed first, so the tile is (2 (2 big)) + 2 (2^-7)
    want0 = (f(2 * big) + f(2 * big)) + (f(2 * small) + f(2 * small))
    assert stats[0, 0, 0, 0] == want0 == f(4 * big + 4 * small)
    # tile 1, coordinate 1: T0 = 2 big (per token) and T2 = T3 = 2^-8 per token
    t0 = f(2 * big) + f(2 * big)
    want1 = ((t0 + f(0)) + f(2 * small)) + f(2 * small)
    assert stats[0, 0, 1, 1] == want1
    assert stats[0, 0, 0, 2] == f(6.0)
    # the orders this rules out round differently on the single-token case
    _, one = oracle.s16_step(x[:, :1], dt[:, :1], A, B[:, :1], C[:, :1], D, db, st.copy(), collect_stats=True)
    assert one[0, 0, 0, 0] == two_big + f(2 * small)          # (big + big) + (small + small): exact
    assert ((two_big + f(small)) + f(small)) == two_big        # sequential rows: the ties lose both
    assert one[0, 0, 1, 1] == two_big                          # ((T0 + 0) + small) + small ties back
    assert (two_big + f(0)) + (f(small) + f(small)) != two_big  # a pairwise fold would keep 2^-7
    assert float(one[0, 0, 1, 1]) != 2 * big + 2 * small       # nor is it the float64 sum
