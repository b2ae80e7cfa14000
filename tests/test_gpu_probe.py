"""The device's exact arithmetic primitives against the oracle, exhaustively
where the domain allows (all binary16 and E4M3 patterns, every stored-scale
boundary)."""
import numpy as np
import pytest
import torch

from mamba2_recall import _native

pytestmark = pytest.mark.gpu


def dev_unary(values, op, device):
    v = torch.from_numpy(np.ascontiguousarray(values, np.uint32).view(np.int32)).to(device)
    out = torch.empty_like(v)
    _native.call("m2r_probe_unary", _native.ptr(v), _native.ptr(out), v.numel(), op, _native.stream_of(v))
    return out.cpu().numpy().view(np.uint32)


def floats_sample(rng, n):
    u = rng.integers(0, 2 ** 32, size=n, dtype=np.uint64).astype(np.uint32)
    return u


def same_float_bits(a, b):
    """Bit equality, with every NaN equal to every NaN (payloads are outside
    the codec's contract: scales and states are finite)."""
    fa, fb = a.view(np.float32), b.view(np.float32)
    return (a == b) | (np.isnan(fa) & np.isnan(fb))


def test_f16_conversions(oracle, device):
    every16 = np.arange(65536, dtype=np.uint32)
    assert same_float_bits(dev_unary(every16, 1, device), oracle.unary(every16, 1)).all()
    # every binary16 value, its neighbours in binary32 and all midpoints
    f = every16.astype(np.uint16).view(np.float16).astype(np.float32)
    f = f[np.isfinite(f)]
    mids = ((f[:-1].astype(np.float64) + f[1:]) / 2).astype(np.float32)
    vals = np.concatenate([f, mids, np.nextafter(mids, np.inf), np.nextafter(mids, -np.inf)]).view(np.uint32)
    vals = np.concatenate([vals, floats_sample(np.random.default_rng(1), 1 << 20)])
    assert (dev_unary(vals, 0, device) == oracle.unary(vals, 0)).all()


def test_binary16_reciprocal_is_correctly_rounded(device):
    """The kernels' reciprocal of a stored (binary16) scale: estimate plus one
    Newton step.  Exhaustive over every positive finite binary16 value; the
    reference is IEEE binary32 division."""
    bits = np.arange(1, 0x7C00, dtype=np.uint32)
    s = bits.astype(np.uint16).view(np.float16).astype(np.float32)
    want = (np.float32(1.0) / s).astype(np.float32).view(np.uint32)
    got = dev_unary(bits, 8, device)
    bad = np.nonzero(got != want)[0]
    assert bad.size == 0, f"{bad.size} mismatches, first at f16 0x{int(bits[bad[0]]):04x}"


def test_e4m3_conversions(oracle, device):
    every8 = np.arange(256, dtype=np.uint32)
    assert same_float_bits(dev_unary(every8, 3, device), oracle.unary(every8, 3)).all()
    fin = every8[(every8 & 0x7F) != 0x7F]
    f = oracle.unary(fin, 3).view(np.float32)
    f = np.sort(np.unique(f[np.isfinite(f)]))
    mids = ((f[:-1].astype(np.float64) + f[1:]) / 2).astype(np.float32)
    vals = np.concatenate([f, mids, np.nextafter(mids, np.inf), np.nextafter(mids, -np.inf)])
    rnd = np.random.default_rng(2).uniform(-448, 448, size=1 << 20).astype(np.float32)
    tiny = np.random.default_rng(3).uniform(-0.02, 0.02, size=1 << 18).astype(np.float32)
    vals = np.concatenate([vals, rnd, tiny, [0.0, -0.0]]).astype(np.float32).view(np.uint32)
    assert (dev_unary(vals, 2, device) == oracle.unary(vals, 2)).all()


def test_e4m3_fp8_instructions(oracle, device):
    """The FP8 instructions the state step uses for the latent bytes: decode
    of every code bit for bit (NaN codes included: 0x7F is the positive
    NaN), encode of non-NaN |x| <= 448 against the software conversion at
    every code, every rounding midpoint and their binary32 neighbours, every
    61st binary32 pattern of the range, binary32 subnormals and signed
    zeros."""
    every8 = np.arange(256, dtype=np.uint32)
    got = dev_unary(every8, 9, device)
    want = oracle.unary(every8, 3)
    assert (got == want).all(), [hex(int(c)) for c in every8[got != want]]
    fin = every8[(every8 & 0x7F) != 0x7F]
    f = oracle.unary(fin, 3).view(np.float32)
    f = np.sort(np.unique(f))
    mids = ((f[:-1].astype(np.float64) + f[1:]) / 2).astype(np.float32)
    near = np.concatenate([f, mids]).view(np.uint32).astype(np.int64)
    near = np.concatenate([near + d for d in range(-4, 5)])
    near = near[(near >= 0) & (near < 2 ** 32)].astype(np.uint32)
    sweep = np.arange(0, 0x43E00001, 61, dtype=np.uint32)
    vals = np.concatenate([near, sweep, sweep | 0x80000000, np.arange(1, 4096, dtype=np.uint32),
                           np.array([0, 0x80000000, 0x43E00000, 0xC3E00000], np.uint32)])
    vals = vals[np.abs(vals.view(np.float32)) <= 448.0]
    got = dev_unary(vals, 10, device)
    want = oracle.unary(vals, 2)
    bad = np.nonzero(got != want)[0]
    assert bad.size == 0, f"{bad.size} mismatches, first at 0x{int(vals[bad[0]]):08x}"


def test_round_and_transcendentals(oracle, device):
    rng = np.random.default_rng(4)
    vals = np.concatenate([floats_sample(rng, 1 << 20),
                           (np.arange(-600, 600) / 2).astype(np.float32).view(np.uint32)])
    assert (dev_unary(vals, 4, device) == oracle.unary(vals, 4)).all()
    args = np.concatenate([rng.uniform(-120, 30, size=1 << 20), rng.normal(0, 3, size=1 << 18)]).astype(np.float32)
    assert (dev_unary(args.view(np.uint32), 5, device) == oracle.unary(args.view(np.uint32), 5)).all()
    logs = np.concatenate([rng.uniform(1, 5e8, size=1 << 19), 1 + rng.uniform(0, 1, size=1 << 19)]).astype(np.float32)
    assert (dev_unary(logs.view(np.uint32), 6, device) == oracle.unary(logs.view(np.uint32), 6)).all()
    sp = np.concatenate([rng.normal(0, 4, size=1 << 20), [20.0, 20.000002, 19.999998, -30, 0]]).astype(np.float32)
    assert (dev_unary(sp.view(np.uint32), 7, device) == oracle.unary(sp.view(np.uint32), 7)).all()


@pytest.mark.parametrize("limit", [7, 127])
def test_stored_quantize_every_scale_boundary(oracle, device, limit):
    """Every positive FP16 scale (plus zero and the largest), values at every
    half-integer boundary k+1/2 (and +-1 ulp) and random values."""
    s_bits = np.arange(0, 0x7C00, 3, dtype=np.uint16)
    s = s_bits.view(np.float16).astype(np.float32)
    ks = np.arange(0, limit + 2, dtype=np.float32) + 0.5
    v = (s[:, None] * ks[None, :]).astype(np.float32)
    vals = np.concatenate([v.ravel(), np.nextafter(v, np.inf).ravel(), np.nextafter(v, -np.inf).ravel()])
    scales = np.tile(np.repeat(s_bits, ks.size), 3)
    vals = np.concatenate([vals, -vals])
    scales = np.concatenate([scales, scales])
    # non-finite values and scales: zero, negative, infinite and NaN scales
    # against finite, infinite and NaN values
    sp_s = np.array([0x0000, 0x8000, 0x3C00, 0xBC00, 0x7C00, 0xFC00, 0x7E00], np.uint16)
    sp_v = np.array([0.0, 1.0, -3.5, np.inf, -np.inf, np.nan], np.float32)
    vals = np.concatenate([vals, np.tile(sp_v, sp_s.size)])
    scales = np.concatenate([scales, np.repeat(sp_s, sp_v.size)])
    want = oracle.stored_quantize(vals, scales, limit)
    vd = torch.from_numpy(vals).to(device)
    sd = torch.from_numpy(scales.view(np.int16)).to(device)
    q = torch.empty(vals.size, dtype=torch.int32, device=device)
    _native.call("m2r_probe_stored_quantize", _native.ptr(vd), _native.ptr(sd), _native.ptr(q), vals.size, limit,
                 _native.stream_of(vd))
    assert (q.cpu().numpy() == want).all()


def test_butterfly_levels_and_pair_tree(device):
    """Each butterfly level adds the xor partner's value, and the wave tree
    equals the canonical adjacent-pair tree (bit-exact)."""
    lanes = np.arange(64, dtype=np.float32)
    vals = np.random.default_rng(9).standard_normal(128).astype(np.float32)
    inp = torch.from_numpy(np.concatenate([lanes, vals])).to(device)
    out = torch.empty(386, dtype=torch.float32, device=device)
    _native.call("m2r_probe_butterfly", _native.ptr(inp), _native.ptr(out), _native.stream_of(inp))
    o = out.cpu().numpy()
    ln = np.arange(64)
    # levels 2 and 3 are mirrors inside the (half-)row: the partner lies in the
    # other aligned half-block, which is all the tree needs
    expect = {0: ln ^ 1, 1: ln ^ 2, 2: (ln & ~7) | (7 - (ln & 7)), 3: (ln & ~15) | (15 - (ln & 15)),
              4: ln ^ 16, 5: ln ^ 32}
    got = {lv: (o[lv * 64:(lv + 1) * 64] - lanes).astype(np.int64) for lv in range(6)}
    for level in range(6):
        assert (got[level] == expect[level]).all(), (level, got[level].tolist())

    def tree(v):
        v = v.copy()
        while v.size > 1:
            v = (v[0::2] + v[1::2]).astype(np.float32)
        return v[0]
    assert o[384].view(np.uint32) == tree(vals).view(np.uint32)
    assert o[385].view(np.uint32) == tree(lanes).view(np.uint32)
