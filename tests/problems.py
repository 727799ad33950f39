"""Problem builders shared by the CPU and GPU tests (test infrastructure only)."""
import numpy as np

from lowbit_amd import formats as F


def outlier_int4_problem(rng, m: int, n: int, k: int, amp: float = 1e6, per_row: int = 3):
    """Activations with a few huge entries where every weight row's code equals its
    group's zero-point (a dequantized weight of exactly 0), asymmetric int4 weights
    otherwise random. The reference's W4A16 bound, 1e-5 * (|X| @ |W|^T), takes nothing
    from those entries, while a kernel that forms sum q x - z sum x rounds partial sums
    of size z * amp: this separates the two formulations.

    Returns (x [m, k] float32, W Int4Weights)."""
    w = rng.standard_normal((n, k)).astype(np.float32)
    W = F.quantize_int4(w, asym=True)
    codes = W.codes()
    z = np.repeat(W.zeros, W.group, axis=1)[:, :W.kp]
    x = rng.standard_normal((m, k)).astype(np.float32)
    for i in range(m):
        cols = rng.choice(k, size=per_row, replace=False)
        x[i, cols] = amp * rng.choice([-1.0, 1.0], size=per_row)
        codes[:, cols] = z[:, cols]
    W = F.Int4Weights(F.pack_nibbles(codes.astype(np.uint8), W.group), W.scales, W.zeros, W.k, W.group)
    # the zero-point codes must be large where the outliers sit, or both forms agree
    assert (z >= 8).mean() > 0.3
    return x, W
