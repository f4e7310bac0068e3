"""Comparison bars of the encoder-block parity tests, and the oracle's block
compositions (oracle/blocks.py) re-exported for the tests that import them
from here."""
import numpy as np

from oracle.blocks import (_attention, _mm, axial_cis, gelu_ref, gelu_tanh, hiera_block_ref, hiera_win_part,  # noqa: F401
                           hiera_win_unpart, ln_ref, maxpool2, rope_ref, vit_block_ref, vit_block_rows, vit_qkv,
                           win_part, win_rows, win_unpart)


# ---------------------------------------------------------------- comparison statistics
def rms(a):
    return float(np.sqrt((np.asarray(a, dtype=np.float64) ** 2).mean()))


def block_stats(got, ref16, ref32):
    d16, d32, spread = np.abs(got - ref16), np.abs(got - ref32), np.abs(ref16 - ref32)
    return d16, d32, spread, (f"max16 {d16.max():.2e} rms16 {rms(d16):.2e} max32 {d32.max():.2e} "
                              f"rms32 {rms(d32):.2e} oracle spread max {spread.max():.2e} rms {rms(spread):.2e}")


def mean_t(d, axis):
    """max over columns (axis 0) or rows (axis 1) of |mean| / standard error,
    each line against its own spread (rows differ in how many flipped
    roundings they received)."""
    n = d.shape[axis]
    se = np.sqrt((d ** 2).mean(axis=axis) / n)
    return float((np.abs(d.mean(axis=axis)) / np.maximum(se, 1e-30)).max())


def block_bars(got, ref16, ref32, what):
    """The block parity bars against the two oracle runs (fp16-rounded Q/K/V
    evaluated exactly, and ggml-cpu's F32 attention), whose own spread is the
    noise floor of two legitimate implementations:
    - max |gpu - ref| <= max(1e-2, 1.5 * spread max) for both runs (1e-2: the
      reference's CPU-vs-GPU block bound, tests/test_metal_overhead.cpp:
      240-246; 1.5: the max of many elements varies ~15% between noise
      realisations);
    - RMS |gpu - ref| <= max(5e-4, 1.25 * spread RMS);
    - every column mean and row mean of (gpu - ref16) within 6 standard
      errors of zero: flipped roundings are symmetric, while a systematic
      error (a missing bias, a wrong row map, a scale) shifts whole lines."""
    d16, d32, spread, stats = block_stats(got, ref16, ref32)
    max_bar = max(1e-2, 1.5 * float(spread.max()))
    rms_bar = max(5e-4, 1.25 * rms(spread))
    s16 = got.astype(np.float64) - ref16
    col, row = mean_t(s16, 0), mean_t(s16, 1)
    stats += f"; bars max {max_bar:.2e} rms {rms_bar:.2e}; worst column / row mean {col:.1f} / {row:.1f} std. errors"
    print(f"{what}: {got.shape[0]} rows, {stats}", flush=True)
    assert d16.max() <= max_bar and d32.max() <= max_bar, f"{what}: {stats}"
    assert rms(d16) <= rms_bar and rms(d32) <= rms_bar, f"{what}: {stats}"
    assert col <= 6.0 and row <= 6.0, f"{what}: {stats}"
    return float(spread.max()), rms(spread)
