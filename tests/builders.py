"""Model builders shared by the tests (host side, numpy).

norm_raw: an RMSNorm weight vector of 1 + 0.3 N(0, 1) values, so that a norm
applied with the wrong vector (attn_norm for ffn_norm, layer l for l + 1, or
not at all) changes the logits.

q_rows: `rows` quantised rows of `cols` N(0, std) weights in dtype `dt`.
Large tensors quantise `unique` random rows on the host and repeat them;
repeat r of a row has its nb blocks in reverse order when r // (2 nb) is
odd, then rotated by r % nb positions along the row, its values negated (the
signs of the block's fp16 scale and min fields flipped) when r // nb is odd,
and its block scales moved by (r // (4 nb)) % 8 fp16 ulps, so that rows a
multiple of `unique` apart are different weight vectors (not the same row at
a slightly different scale) and a row or tile index error of that stride
changes the result as any other does.  The scale moves by at most 7 ulps
(0.7 %): a larger move of d without dmin would give the row a mean far from
zero, and logits that amplify every rounding difference of the hidden state.
"""
import numpy as np

import pyoracle as P

# byte offset of the fp16 scale inside one block, and the block size
SCALE_AT = {P.Q4_0: (0, 18), P.Q4_1: (0, 20), P.Q8_0: (0, 34), P.Q4_K: (0, 144),
            P.Q6_K: (208, 210)}
# the fp16 fields of one block whose signs flipped together negate the
# block's every value (d and, for the formats with one, the min / offset)
SIGNS_AT = {P.Q4_0: (0,), P.Q4_1: (0, 2), P.Q8_0: (0,), P.Q4_K: (0, 2), P.Q6_K: (208,)}


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
        blocks = raw.reshape(rows, nb, bb)
        for r in range(1, reps):
            sl = slice(r * u, min((r + 1) * u, rows))
            b = blocks[sl]
            if (r // (2 * nb)) % 2 == 1:
                b = b[:, ::-1]
            b = np.roll(b, r % nb, axis=1)
            if (r // nb) % 2 == 1:
                for off in SIGNS_AT[dt]:
                    b[:, :, off + 1] ^= 0x80
            blocks[sl] = b
        d = raw.reshape(rows, nb, bb)[:, :, at:at + 2].copy().view(np.uint16)[..., 0]
        bump = ((np.arange(rows) // u // (4 * nb)) % 8).astype(np.uint16)[:, None]
        # a finite positive or negative fp16 moves by a few ulps (zeros stay)
        d = np.where((d & 0x7FFF) != 0, d + bump, d).astype(np.uint16)
        blk = raw.reshape(rows, nb, bb)
        blk[:, :, at:at + 2] = d[..., None].view(np.uint8).reshape(rows, nb, 2)
    return dict(raw=np.ascontiguousarray(raw).ravel(), dtype=dt, ne0=cols, ne1=rows)
