"""Seeded parity sweep of the state steps (ridge, tier, legacy, dense3 and
the FP16-carry control) against the C oracle: every published layout at batch 1 to 64 (every
workgroup shape the launch picks:
four and two waves per slot, one slot per wave, four slots per wave), one and
three tokens, head dimensions 48, 64 and 80, D / dt_bias in binary16 and
binary32, and inputs and stored scales over several decades.  Packed codes,
scales and latent bytes bit-exact; y within the north_star tolerance."""
import pytest

from cases import RIDGE_LAYOUTS, TIER_LAYOUTS
from test_gpu_state import run_ridge, run_tier

pytestmark = pytest.mark.gpu

BATCHES = (1, 2, 3, 8, 16, 64)
X_SCALES = (1.0, 30.0, 1e-3)
SCALE_MUS = (-4.0, -9.0, 0.0)
HEAD_DIMS = (64, 64, 80, 48)


def _case(seed):
    return X_SCALES[seed % 3], SCALE_MUS[(seed // 3) % 3], HEAD_DIMS[seed % 4]


@pytest.mark.parametrize("batch", BATCHES)
@pytest.mark.parametrize("L", (1, 3))
def test_ridge_sweep(oracle, device, batch, L):
    for k, layout in enumerate(RIDGE_LAYOUTS):
        seed = 7000 + 100 * batch + 10 * L + k
        xs, mu, P = _case(seed)
        run_ridge(oracle, device, layout, batch, L, 128, P, 8, seed, x_scale=xs, scale_mu=mu,
                  d_f32=bool(seed % 2), db_f32=bool(seed % 3 == 0))


@pytest.mark.parametrize("batch", BATCHES)
def test_tier_and_legacy_sweep(oracle, device, batch):
    for k, layout in enumerate(TIER_LAYOUTS):
        seed = 8000 + 100 * batch + k
        xs, mu, P = _case(seed)
        kind = "legacy" if k == 0 else "tier"
        run_tier(oracle, device, kind, "16_64_48" if kind == "legacy" else layout, batch, 1 + (seed % 3), 128, P, 8,
                 seed, x_scale=xs, scale_mu=mu, d_f32=bool(seed % 2))


@pytest.mark.parametrize("batch", BATCHES)
@pytest.mark.parametrize("kind", ("permutation", "equalizer"))
def test_dense3_sweep(oracle, device, batch, kind):
    from test_gpu_state import run_dense3
    for L in (1, 2):
        seed = 9500 + 100 * batch + 10 * L + (kind == "equalizer")
        xs, _, P = _case(seed)
        mu = (-2.0, -6.0, 1.0)[(seed // 3) % 3]
        # inputs 30x the unit scale can overflow y (binary16) on both sides:
        # then finite rows and the NaN / infinite pattern are compared
        run_dense3(oracle, device, kind, batch, L, 128, P, 8, seed, x_scale=xs, scale_mu=mu, nonfinite_y=xs > 1)


@pytest.mark.parametrize("batch", BATCHES)
def test_s16_sweep(oracle, device, batch):
    """FP16-carry step: carry and statistics bit-exact (one fixed summation
    order), y within tolerance; ragged P included."""
    from test_gpu_state import run_s16
    for L in (1, 3):
        seed = 9800 + 100 * batch + L
        P = HEAD_DIMS[seed % 4] - (8 if seed % 3 == 0 else 0)
        run_s16(oracle, device, batch, L, 128, P, 8, seed, collect=bool(seed % 2))
