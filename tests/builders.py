"""Model builders shared by the tests (host side, numpy).

norm_raw: an RMSNorm weight vector of 1 + 0.3 N(0, 1) values, so that a norm
applied with the wrong vector (attn_norm for ffn_norm, layer l for l + 1, or
not at all) changes the logits.

q_rows: `rows` quantised rows of `cols` N(0, std) weights in dtype `dt`.
Large tensors quantise `unique` random rows on the host and repeat them; each
repeat's block scales are then moved by a few fp16 ulps per repeat, so that no
two rows of the tensor are equal and a row or tile index error shows in the
result.
"""
import numpy as np

import pyoracle as P

# byte offset of the fp16 scale inside one block, and the block size
SCALE_AT = {P.Q4_0: (0, 18), P.Q4_1: (0, 20), P.Q8_0: (0, 34), P.Q4_K: (0, 144),
            P.Q6_K: (208, 210)}


def norm_raw(rng, n):
    w = (1.0 + 0.3 * rng.standard_normal(n)).astype(np.float32)
    return dict(raw=w.view(np.uint8).copy(), dtype=P.F32, ne0=n, ne1=1)


def q_rows(orc, rng, rows, cols, dt, std=0.02, unique=2048):
    u = min(rows, unique)
    w = (rng.standard_normal((u, cols)) * std).astype(np.float32)
    one = orc.quantize(w, dt).reshape(u, -1)
    reps = -(-rows // u)
    raw = np.tile(one, (reps, 1))[:rows].copy()
    if reps > 1 and dt in SCALE_AT:
        at, bb = SCALE_AT[dt]
        nb = raw.shape[1] // bb
        d = raw.reshape(rows, nb, bb)[:, :, at:at + 2].copy().view(np.uint16)[..., 0]
        bump = (np.arange(rows) // u).astype(np.uint16)[:, None] * 3
        # a finite positive or negative fp16 moves by a few ulps (zeros stay)
        d = np.where((d & 0x7FFF) != 0, d + bump, d).astype(np.uint16)
        blk = raw.reshape(rows, nb, bb)
        blk[:, :, at:at + 2] = d[..., None].view(np.uint8).reshape(rows, nb, 2)
    return dict(raw=np.ascontiguousarray(raw).ravel(), dtype=dt, ne0=cols, ne1=rows)
