"""GPU parity of the FP4 decode kernels against the CPU oracle: FP16 bits
bit-exact, and the reference's ValueError conditions raised in its order."""
import numpy as np
import pytest
import torch

import cases

pytestmark = pytest.mark.gpu


def g16_packet(rng, rows, cols, device, *, global_scale=None):
    """Random nibbles; block scales per the BASELINE recipe: s ~ lognormal(-3,
    0.5), global = max(s)/448, block byte = E4M3(clamp(s/global, 0, 448))."""
    groups = (cols + 15) // 16
    packed = rng.integers(0, 256, size=(rows, groups * 8), dtype=np.uint16).astype(np.uint8)
    if cols % 16:
        # zero the padding nibbles of the final group
        codes = np.stack((packed & 15, packed >> 4), -1).reshape(rows, -1)
        codes[:, cols:] = 0
        packed = (codes[:, 0::2] | (codes[:, 1::2] << 4)).astype(np.uint8)
    s = np.exp(rng.normal(-3.0, 0.5, size=(rows, groups))).astype(np.float32)
    g = np.float32(s.max() / 448.0) if global_scale is None else np.float32(global_scale)
    sb = torch.from_numpy(np.clip(s / g, 0, 448)).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    return packed, sb, g


def decode_dev(packed, scales_u8, g, rows, cols, device, group=16):
    from mamba2_recall import fp4
    pk = torch.from_numpy(packed).to(device)
    if group == 16:
        sc = torch.from_numpy(scales_u8).to(device).view(torch.float8_e4m3fn)
        packet = dict(format="fp4_g16_e4m3", shape=[rows, cols], group_size=16, packed=pk, scales=sc,
                      global_scale=torch.tensor(g, dtype=torch.float32))
    else:
        sc = torch.from_numpy(scales_u8.view(np.float16)).to(device)
        packet = dict(format="fp4_g64_f16", shape=[rows, cols], group_size=64, packed=pk, scales=sc,
                      global_scale=None)
    return fp4.decode_packet(packet)


# (33, 4112): 16 whole blocks of 1024 units for the wide-load kernel and 578 units for the per-unit one
@pytest.mark.parametrize("rows,cols", [(512, 4096), (37, 8192), (33, 4112), (3, 48), (5, 40)])
def test_g16_random_bit_exact(oracle, device, rows, cols):
    rng = np.random.default_rng(rows * 7 + cols)
    packed, sb, g = g16_packet(rng, rows, cols, device)
    print(f"[fp4 g16] rows={rows} cols={cols}", flush=True)
    want, err = oracle.fp4_decode(16, packed, sb, g, rows, cols)
    assert err == 0
    got = decode_dev(packed, sb, g, rows, cols, device).cpu().numpy().view(np.uint16)
    assert int((got != want).sum()) == 0


def test_g16_every_code_every_scale_byte(oracle, device):
    """All 16 codes x all 254 finite non-negative-or-zero scale bytes x a set
    of globals, including ones that overflow FP16 (must raise)."""
    scale_bytes = np.array([b for b in range(256) if (b & 0x7F) != 0x7F and (b < 0x80 or b == 0x80)], np.uint8)
    codes = np.arange(16, dtype=np.uint8)
    for g in (1.0, 2.0 ** -20, 0.3, 1.7e-3, 100.0, 2.0 ** 24):
        rows = scale_bytes.size
        cols = 16 * 16
        code_mat = np.tile(np.repeat(codes, 16), (rows, 1))              # group j holds code j
        sb = np.repeat(scale_bytes[:, None], 16, axis=1)                  # [rows, 16 groups]
        # zero scale bytes may only hold codes 0/8: keep those rows' other groups at code 0
        zero_rows = (scale_bytes & 0x7F) == 0
        code_mat[zero_rows] = np.where(np.isin(code_mat[zero_rows], (0, 8)), code_mat[zero_rows], 0)
        packed = (code_mat[:, 0::2] | (code_mat[:, 1::2] << 4)).astype(np.uint8)
        want, err = oracle.fp4_decode(16, packed, sb, g, rows, cols)
        print(f"[fp4 g16 KAT] global={g} err={err}", flush=True)
        if err:
            assert err == 8, err
            with pytest.raises(ValueError, match="Nonfinite decoded FP16 weights"):
                decode_dev(packed, sb, g, rows, cols, device)
            continue
        got = decode_dev(packed, sb, g, rows, cols, device).cpu().numpy().view(np.uint16)
        assert int((got != want).sum()) == 0
        # closed form: FP16(FP32(FP32(lev*sign*block)*global)) via numpy float32
        lev = np.array([0, .5, 1, 1.5, 2, 3, 4, 6], np.float32)
        blk = torch.from_numpy(sb).view(torch.float8_e4m3fn).float().numpy()
        c = code_mat.reshape(rows, 16, 16)
        val = (lev[c & 7] * np.where(c & 8, np.float32(-1), np.float32(1))).astype(np.float32)
        val = (val * blk[:, :, None]).astype(np.float32) * np.float32(g)
        closed = val.astype(np.float32).astype(np.float16).view(np.uint16).reshape(rows, cols)
        assert int((closed != got).sum()) == 0


def _assert_equal_in_chunks(got_dev, want, rows_per_chunk=16384):
    for r0 in range(0, want.shape[0], rows_per_chunk):
        got = got_dev[r0:r0 + rows_per_chunk].cpu().numpy().view(np.uint16)
        bad = int((got != want[r0:r0 + rows_per_chunk]).sum())
        assert bad == 0, f"rows {r0}..: {bad} mismatched FP16 weights"


def test_g16_embedding_matrix_bit_exact(oracle, device):
    """The [256000, 4096] embedding / lm_head matrix of the full 8B set
    (131,072,000 eight-weight units) at the automatic decode shape: one pass
    of 128,000 workgroups."""
    rows, cols = 256000, 4096
    rng = np.random.default_rng(256000)
    packed = rng.integers(0, 256, size=(rows, cols // 2), dtype=np.uint8)
    s = np.exp(rng.normal(-3.0, 0.5, size=(rows, cols // 16))).astype(np.float32)
    g = np.float32(s.max() / 448.0)
    sb = torch.from_numpy(np.clip(s / g, 0, 448)).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    del s
    print(f"[fp4 g16 embedding] rows={rows} cols={cols} units={rows * cols // 8}", flush=True)
    want, err = oracle.fp4_decode(16, packed, sb, g, rows, cols)
    assert err == 0
    _assert_equal_in_chunks(decode_dev(packed, sb, g, rows, cols, device), want)


def _forced_fp4_shape(upt, cap, nt):
    from mamba2_recall import _native
    lib = _native.lib()
    assert lib.m2r_set_fp4_decode_shape(upt, cap, nt) == 0
    return lib


@pytest.mark.parametrize("upt,cap,nt", [(1, 2048, 1), (2, 4096, 0), (4, 2048, 1), (4, 0, 0), (8, 1024, 0),
                                        (8, 0, 1)])
def test_g16_forced_shapes_and_grid_stride_sweeps(oracle, device, upt, cap, nt):
    """Every decode shape the tuning hook offers gives the oracle's weights:
    1-8 units per thread, default and non-temporal stores, and grid caps of
    1024-4096 workgroups, which make each workgroup stride over the
    [4096, 8192] out_proj matrix (4,194,304 units) in 2 to 16 sweeps."""
    rows, cols = 4096, 8192
    rng = np.random.default_rng(upt * 100 + cap + nt)
    packed = rng.integers(0, 256, size=(rows, cols // 2), dtype=np.uint8)
    s = np.exp(rng.normal(-3.0, 0.5, size=(rows, cols // 16))).astype(np.float32)
    g = np.float32(s.max() / 448.0)
    sb = torch.from_numpy(np.clip(s / g, 0, 448)).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    print(f"[fp4 g16 shape] upt={upt} cap={cap} nt={nt}", flush=True)
    want, err = oracle.fp4_decode(16, packed, sb, g, rows, cols)
    assert err == 0
    lib = _forced_fp4_shape(upt, cap, nt)
    try:
        got = decode_dev(packed, sb, g, rows, cols, device)
    finally:
        lib.m2r_set_fp4_decode_shape(0, 0, 1)
    _assert_equal_in_chunks(got, want)


def test_g64_grid_stride_sweeps(oracle, device):
    """G64 under a forced grid cap of 2048 workgroups: 20,480,000 units in
    ten sweeps."""
    rows, cols = 40000, 4096
    rng = np.random.default_rng(40000)
    packed = rng.integers(0, 256, size=(rows, cols // 2), dtype=np.uint8)
    sc = np.exp(rng.normal(-3.0, 0.5, size=(rows, cols // 64))).astype(np.float16).view(np.uint16)
    print(f"[fp4 g64 sweeps] rows={rows} cols={cols} units={rows * cols // 8}", flush=True)
    want, err = oracle.fp4_decode(64, packed, sc, 1.0, rows, cols)
    assert err == 0
    lib = _forced_fp4_shape(4, 2048, 1)
    try:
        got = decode_dev(packed, sc, None, rows, cols, device, group=64)
    finally:
        lib.m2r_set_fp4_decode_shape(0, 0, 1)
    _assert_equal_in_chunks(got, want)
    _assert_equal_in_chunks(decode_dev(packed, sc, None, rows, cols, device, group=64), want)


# (19, 8256): 19 whole blocks of 1024 units for the wide-load kernel and 152 units for the per-unit one
@pytest.mark.parametrize("rows,cols", [(64, 4096), (19, 8256), (7, 192), (3, 100)])
def test_g64_random_bit_exact(oracle, device, rows, cols):
    rng = np.random.default_rng(rows + cols)
    groups = (cols + 63) // 64
    codes = rng.integers(0, 16, size=(rows, groups * 64)).astype(np.uint8)
    codes[:, cols:] = 0
    packed = (codes[:, 0::2] | (codes[:, 1::2] << 4)).astype(np.uint8)
    sc = np.exp(rng.normal(-3.0, 0.5, size=(rows, groups))).astype(np.float16).view(np.uint16)
    print(f"[fp4 g64] rows={rows} cols={cols}", flush=True)
    want, err = oracle.fp4_decode(64, packed, sc, 1.0, rows, cols)
    assert err == 0
    got = decode_dev(packed, sc, None, rows, cols, device, group=64).cpu().numpy().view(np.uint16)
    assert int((got != want).sum()) == 0


def test_decode_errors_follow_reference_order(device):
    rng = np.random.default_rng(5)
    rows, cols = 4, 64
    packed, sb, g = g16_packet(rng, rows, cols, device)
    bad = sb.copy(); bad[1, 2] = 0x7F                        # NaN block scale
    with pytest.raises(ValueError, match="Invalid stored scale"):
        decode_dev(packed, bad, g, rows, cols, device)
    bad = sb.copy(); bad[0, 0] = 0xB8                        # negative block scale
    with pytest.raises(ValueError, match="Invalid stored scale"):
        decode_dev(packed, bad, g, rows, cols, device)
    with pytest.raises(ValueError, match="Global scale must be finite and positive"):
        decode_dev(packed, sb, 0.0, rows, cols, device)
    bad = sb.copy(); bad[2, 1] = 0x00                        # zero block with nonzero codes
    pk = packed.copy(); pk[2, 8:16] = 0x31
    with pytest.raises(ValueError, match="Nonzero code in a zero-scale group"):
        decode_dev(pk, bad, g, rows, cols, device)
    pk = packed.copy(); pk[2, 8:16] = 0x88                   # codes 8 (= -0) are allowed
    out = decode_dev(pk, bad, g, rows, cols, device).cpu().numpy().view(np.uint16)
    assert (out[2, 16:32] == 0x8000).all()
    p2, s2, g2 = g16_packet(rng, 2, 40, device)
    p2[:, -1] |= 0x30                                         # padding nibble (column 41) nonzero
    with pytest.raises(ValueError, match="Nonzero final-group padding"):
        decode_dev(p2, s2, g2, 2, 40, device)


@pytest.mark.parametrize("M,N,K", [(1, 18560, 4096), (2, 1000, 4096), (4, 333, 4096), (1, 4096, 8192),
                                   (2, 257, 8192), (4, 101, 8192), (1, 100, 2048), (4, 63, 2048), (1, 1, 4096)])
def test_fp4_gemv_matches_decoded_weights(device, M, N, K):
    """fp4.gemv_g16 (packed-resident FP4 G16 GEMV) against the product with
    the decoded FP16 weights (decode_packet, bit-exact to the oracle) in
    float64: relative L2 <= 1e-3 (north_star tolerance), and every output
    within one binary16 ulp plus the binary32 accumulation bound K * 2^-22 *
    sum|u w|.  Packets in the reference G16 format, with some zero-scale
    groups holding codes 0 and 8."""
    import torch
    from mamba2_recall import fp4
    gen = torch.Generator(device=device).manual_seed(M * 7919 + N)
    print(f"[fp4 gemv] M={M} N={N} K={K}", flush=True)
    packed = torch.randint(0, 256, (N, K // 2), generator=gen, device=device, dtype=torch.uint8)
    s = torch.exp(torch.randn((N, K // 16), generator=gen, device=device) * 0.5 - 3.0)
    g = (s.max() / 448.0).float().reshape(1)
    sb = (s / g).clamp(0, 448).to(torch.float8_e4m3fn).view(torch.uint8)
    zero = torch.rand((N, K // 16), generator=gen, device=device) < 0.02
    sb = torch.where(zero, torch.zeros_like(sb), sb)
    codes = packed.view(N, K // 16, 8)
    codes = torch.where(zero[..., None], codes & 0x88, codes).view(N, K // 2)
    w = fp4.decode_packet(dict(format="fp4_g16_e4m3", shape=[N, K], group_size=16, packed=codes,
                               scales=sb.view(torch.float8_e4m3fn), global_scale=g.reshape(())))
    u = torch.randn((M, K), generator=gen, device=device).half()
    y = fp4.gemv_g16(codes, sb, g, u)
    ref = u.double() @ w.double().T
    torch.cuda.synchronize()
    err = (y.double() - ref).norm() / ref.norm()
    assert float(err) <= 1e-3, float(err)
    bound = (ref.abs() * 2.0 ** -11 + (u.double().abs() @ w.double().abs().T) * K * 2.0 ** -22 + 2.0 ** -24)
    assert bool(((y.double() - ref).abs() <= bound).all())


@pytest.mark.parametrize("N,K", [(18560, 4096), (4640, 4096), (4096, 8192), (2048, 8192), (100, 2048)])
def test_fp4_gemv_one_row_same_bits_as_two_rows(device, N, K):
    """One activation row runs the whole-row kernel where it fills the chip in
    one resident round (in_proj and out_proj shapes of the 8B model), several
    rows the general kernel; both add each row's 2048-wide chunk sums (wave
    sums) in chunk order, so y of one row equals row 0 of the same row passed
    twice, bit for bit."""
    from mamba2_recall import fp4
    gen = torch.Generator(device=device).manual_seed(N + K)
    print(f"[fp4 gemv one row] N={N} K={K}", flush=True)
    codes = torch.randint(0, 256, (N, K // 2), generator=gen, device=device, dtype=torch.uint8)
    s = torch.exp(torch.randn((N, K // 16), generator=gen, device=device) * 0.5 - 3.0)
    g = (s.max() / 448.0).float().reshape(1)
    sb = (s / g).clamp(0, 448).to(torch.float8_e4m3fn).view(torch.uint8)
    u = torch.randn((1, K), generator=gen, device=device).half()
    y1 = fp4.gemv_g16(codes, sb, g, u)
    y2 = fp4.gemv_g16(codes, sb, g, torch.cat((u, u)))
    torch.cuda.synchronize()
    assert torch.equal(y1[0].view(torch.int16), y2[0].view(torch.int16))
    assert torch.equal(y2[0].view(torch.int16), y2[1].view(torch.int16))
