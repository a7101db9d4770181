"""Host restatements of the FRAG16 weight order (include/tau_moe.h) used as the
checker for tau_moe_pack_weights: a loop over the header's piece formula and a
reshape/permute form; test_host pins the two against each other."""
import numpy as np


def frag16_loop(w):
    """Piece p = (b*(k/32) + c)*64 + lane of expert e holds row 16*b + lane%16,
    columns 32*c + 8*(lane//16) .. +8 (the header's definition, literally)."""
    e_, n, k = (1, *w.shape) if w.ndim == 2 else w.shape
    src = w.reshape(e_, n, k)
    out = np.empty((e_, n * k // 8, 8), dtype=w.dtype)
    for e in range(e_):
        for b in range(n // 16):
            for c in range(k // 32):
                for lane in range(64):
                    p = (b * (k // 32) + c) * 64 + lane
                    r, col = 16 * b + lane % 16, 32 * c + 8 * (lane // 16)
                    out[e, p] = src[e, r, col:col + 8]
    return out.reshape(w.shape)


def frag16_permute(w):
    """Same order by axis permutation: (e, band, row16, kc, quarter, 8) ->
    (e, band, kc, quarter, row16, 8)."""
    e_, n, k = (1, *w.shape) if w.ndim == 2 else w.shape
    v = w.reshape(e_, n // 16, 16, k // 32, 4, 8).transpose(0, 1, 3, 4, 2, 5)
    return np.ascontiguousarray(v).reshape(w.shape)
