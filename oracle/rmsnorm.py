"""CPU restatement of (Skip)SimplifiedLayerNormalization — TEST INFRASTRUCTURE.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s CPU leg may import this module,
and only as the checker; the product path never calls it.

Follows the reference kernel ``rust/shaders/glsl/skip_simplified_layer_norm_f16.comp`` (bound by
``rust/src/ops/common/templates.rs:426-528``; the op rows ``rust/src/ops/norm.rs:53-140``):
the residual ``r = x + skip (+ bias)``, ``y = r / sqrt(mean(r^2) + epsilon) * gamma`` over the
last axis, and the residual sum ``r`` as the node's output slot 3; ``SimplifiedLayerNormalization``
is the same without ``skip``.  Default epsilon 1e-5 (``templates.rs:399``).  Here in float64.

Pinned in ``tests/test_rmsnorm_oracle.py`` against ``torch.nn.functional.rms_norm`` (a library
routine), closed forms (a constant row, scale invariance with epsilon 0, gamma linearity) and a
pure-Python brute force.
"""

from __future__ import annotations

import numpy as np


def skip_rmsnorm(x, gamma, skip=None, bias=None, epsilon: float = 1e-5):
    """``(y, r)`` in float64 over the last axis."""
    r = np.asarray(x, dtype=np.float64)
    if skip is not None:
        r = r + np.asarray(skip, dtype=np.float64)
    if bias is not None:
        r = r + np.asarray(bias, dtype=np.float64)
    ms = np.mean(r * r, axis=-1, keepdims=True)
    y = r / np.sqrt(ms + epsilon) * np.asarray(gamma, dtype=np.float64)
    return y, r


def make_inputs(rows: int, hidden: int, dtype=np.float16, seed: int = 20260801, bias=True):
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((rows, hidden), dtype=np.float32).astype(dtype)
    skip = rng.standard_normal((rows, hidden), dtype=np.float32).astype(dtype)
    gamma = (1.0 + 0.1 * rng.standard_normal(hidden, dtype=np.float32)).astype(dtype)
    b = (0.1 * rng.standard_normal(hidden, dtype=np.float32)).astype(dtype) if bias else None
    return {"x": x, "skip": skip, "gamma": gamma, "bias": b}
