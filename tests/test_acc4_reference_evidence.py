"""accuracy_level = 4 against the only level-4 evidence the reference holds.

The reference records one measurement of ORT's level 4 against level 1 (fp32 accumulation):
``max_abs=3.6e-3, mean_abs=7.5e-4, rtol_max=4.6e-3`` at K=1024, N=512
(``tests/ops/_models.py:55-66``; ``rtol_max = max(|a-b| / (1e-8 + |b|))``,
``_models.py:2693,2719-2726``), made with the inputs of ``make_matmulnbits_model``
(``_models.py:2473-2553``).  Those inputs are fully determined by numpy's
``default_rng(42)``; ``reference_inputs`` below draws them in the same order and shapes
(packed bytes, the fp32 activation row, U(0.001, 0.1) scales, random zero-point bytes).

What this pins, without ORT (absent here and on the GPU box):

* The oracle's level-4 deviation from level 1 is what symmetric per-block int8 quantisation of A
  with step ``amax/127`` and round-to-nearest produces: each activation moves by an error
  uniform in ``[-step/2, step/2]``, so ``y[n]`` moves by a sum of independent terms with variance
  ``sum_k (step_k^2 / 12) * w[n][k]^2``.  The normalised deviations must then have unit mean
  square (K = 1024 terms each; a chi-square bound over the 512 outputs).  A coarser step
  (amax/63), a finer one (amax/255), truncation instead of rounding, or a dropped activation
  scale each miss this by a factor of 4 or more.
* The recorded figures do not come from these inputs: on them ANY per-block 8-bit quantiser
  whose step is ``amax/127`` moves y by ~0.05 on average (the model's prediction, which the
  oracle meets), about 68x the recorded mean.  The test states that gap explicitly, so the
  recorded numbers are never mistaken for a band this oracle should hit; the one scale-free
  figure the record allows, mean_abs / max_abs, is compared instead.

Still unpinned against ORT (``SQNBIT_CompInt8`` source is not available here): the tie rule of
the rounding (half-even here; ties have probability zero for continuous activations), whether the
step multiplies as ``a * (127 / amax)`` or divides as ``a / (amax / 127)`` (a one-ulp difference
that flips an occasional code by one), and the fp32 order in which ``sA * sB * dot`` is formed.
"""

from __future__ import annotations

import numpy as np

from oracle import matmul_nbits as orc

K, N, BITS, BS = 1024, 512, 4, 32
RECORDED = {"max_abs": 3.6e-3, "mean_abs": 7.5e-4, "rtol_max": 4.6e-3}


def reference_inputs():
    """make_matmulnbits_model(K=1024, N=512) defaults: bits 4, block 32, fp32 activations,
    zero points on, rows 1 — drawn from default_rng(42) in the file's order."""
    rng = np.random.default_rng(42)
    bpc = -(-K // BS)
    packed = rng.integers(0, 256, size=[N, bpc, BS * BITS // 8], dtype=np.uint8)
    act = rng.standard_normal((1, K)).astype(np.float32)
    scale = rng.uniform(0.001, 0.1, size=[N * bpc]).astype(np.float32)
    zp_bytes = -(-(bpc * BITS) // 8)
    zp = rng.integers(0, 256, size=[N, zp_bytes], dtype=np.uint8)
    return act, packed, scale, zp


def _stats(y4, y1):
    d = np.abs(y4.astype(np.float64) - y1.astype(np.float64))
    return {"max_abs": float(d.max()), "mean_abs": float(d.mean()),
            "rtol_max": float((d / (1e-8 + np.abs(y1.astype(np.float64)))).max())}


def _predicted_var(act):
    """Variance of y4[n] - y1[n] under uniform rounding error of step amax/127 per block,
    computed from A and the dequantised weights alone (not from the oracle's quantiser)."""
    a = act.reshape(K).astype(np.float64)
    step = np.abs(a.reshape(-1, BS)).max(axis=1) / 127.0
    var_k = np.repeat(step ** 2 / 12.0, BS)                               # [K]
    return var_k


def test_reference_inputs_shapes_match_the_builder():
    act, packed, scale, zp = reference_inputs()
    assert act.shape == (1, K) and act.dtype == np.float32
    assert packed.shape == (N, K // BS, BS // 2)
    assert scale.shape == (N * (K // BS),) and scale.min() >= 0.001 and scale.max() < 0.1
    assert zp.shape == (N, K // BS // 2)


def test_level4_deviation_matches_the_rounding_error_model():
    act, packed, scale, zp = reference_inputs()
    y1 = orc.matmul_nbits(act, packed, scale, zp, N, K, BITS, BS).astype(np.float64)
    y4 = orc.matmul_nbits_acc4(act, packed, scale, zp, N, K, BITS, BS).astype(np.float64)
    w = orc.dequantize_f32(packed, scale, zp, N, K, BITS, BS).astype(np.float64)   # [N, K]
    var = (w ** 2) @ _predicted_var(act)                                           # [N]
    z = (y4 - y1).reshape(N) / np.sqrt(var)
    ms = float(np.mean(z ** 2))
    # chi-square with 512 degrees of freedom: mean 1, sd sqrt(2/512) = 0.0625; +-0.25 is 4 sd
    assert 0.75 <= ms <= 1.25, ms
    # rounding to nearest is unbiased: the mean deviation is within 4 sd of zero
    assert abs(float(np.mean(z))) <= 4.0 / np.sqrt(N), float(np.mean(z))


def test_plausible_quantiser_mistakes_fail_the_model():
    """Planted in a copy of the oracle's quantiser: each mistake moves the mean square of the
    normalised deviations out of the band the correct quantiser meets."""
    act, packed, scale, zp = reference_inputs()
    y1 = orc.matmul_nbits(act, packed, scale, zp, N, K, BITS, BS).astype(np.float64)
    w = orc.dequantize_f32(packed, scale, zp, N, K, BITS, BS).astype(np.float64)
    var = (w ** 2) @ _predicted_var(act)
    a = act.reshape(-1, BS).astype(np.float64)
    amax = np.abs(a).max(axis=1, keepdims=True)

    def ms_of(a_hat):
        y = (a_hat.reshape(1, K) @ w.T).reshape(N)
        return float(np.mean(((y - y1.reshape(N)) / np.sqrt(var)) ** 2))

    good = np.rint(a * (127 / amax)) * (amax / 127)
    coarse = np.rint(a * (63 / amax)) * (amax / 63)
    fine = np.rint(a * (255 / amax)) * (amax / 255)
    trunc = np.trunc(a * (127 / amax)) * (amax / 127)
    assert 0.75 <= ms_of(good) <= 1.25
    for bad in (coarse, fine, trunc):
        m = ms_of(bad)
        assert m > 2.5 or m < 0.4, m


def test_recorded_figures_are_not_from_these_inputs():
    act, packed, scale, zp = reference_inputs()
    y1 = orc.matmul_nbits(act, packed, scale, zp, N, K, BITS, BS)
    y4 = orc.matmul_nbits_acc4(act, packed, scale, zp, N, K, BITS, BS)
    got = _stats(y4, y1)
    w = orc.dequantize_f32(packed, scale, zp, N, K, BITS, BS).astype(np.float64)
    predicted_mean_abs = float(np.mean(np.sqrt(2 / np.pi) * np.sqrt((w ** 2) @ _predicted_var(act))))
    # the oracle meets the model's mean |deviation| ...
    assert abs(got["mean_abs"] / predicted_mean_abs - 1.0) < 0.15, (got, predicted_mean_abs)
    # ... and that is far above every recorded figure: the record was made on other inputs
    for key in ("max_abs", "mean_abs"):
        assert got[key] > 20 * RECORDED[key], (key, got[key], RECORDED[key])
    # the record's only scale-free figure, the ratio of mean to max deviation (0.21), agrees
    rec_ratio = RECORDED["mean_abs"] / RECORDED["max_abs"]
    ratio = got["mean_abs"] / got["max_abs"]
    assert abs(ratio / rec_ratio - 1.0) < 0.3, (ratio, rec_ratio)
