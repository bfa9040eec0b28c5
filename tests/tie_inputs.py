"""Activation rows full of hard rounding ties for the Q8_0 activation kind.

quantize_activations (crates/kf-quant/src/lib.rs:81-140) rounds the f32 product p = v * (1/d) half away from zero.
Values are planted so that p is exactly k + 0.5 in f32 while the exact real product v * id lies just below k + 0.5: a
kernel that rounds the unrounded product (a fused multiply-add inside round's expansion) gives k instead of k + 1.
"""
import numpy as np


def hard_tie_rows(rows: int, n: int, seed: int = 0):
    """(x [rows][n] f32, count of planted ties); every 32-block keeps its largest magnitude, so d is unchanged."""
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((rows, n)).astype(np.float32)
    blocks = x.reshape(rows, n // 32, 32)
    up, down = np.float32(np.inf), np.float32(-np.inf)
    made = 0
    for r in range(rows):
        for g in range(n // 32):
            blk = blocks[r, g]
            top = int(np.abs(blk).argmax())
            amax = np.float32(abs(blk[top]))
            idv = np.float32(1) / np.float32(amax / np.float32(127))
            for slot in range(32):
                if slot == top:
                    continue
                k = int(rng.integers(0, 120))
                sign = np.float32(1 if rng.random() < 0.5 else -1)
                v = np.float32((k + 0.5) / float(idv))
                for _ in range(3):  # walk down a few ulps from the nearest value to (k + 0.5) * d
                    p = np.float32(v * idv)
                    if p == k + 0.5 and float(v) * float(idv) < k + 0.5 and v < amax:
                        blk[slot] = sign * v
                        made += 1
                        break
                    v = np.nextafter(v, down, dtype=np.float32)
                else:
                    v = np.float32((k + 0.5) / float(idv))
                    for _ in range(3):
                        v = np.nextafter(v, up, dtype=np.float32)
                        p = np.float32(v * idv)
                        if p == k + 0.5 and float(v) * float(idv) < k + 0.5 and v < amax:
                            blk[slot] = sign * v
                            made += 1
                            break
    return x, made
