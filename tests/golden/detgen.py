"""Deterministic test inputs from integer arithmetic only (splitmix64), so a
fixture needs just its seed: the same float32 bits on every machine.

values: (sum of four 12-bit uniforms - 8190) / 2048, an approximately normal
variable with sd ~1.15, exactly representable in float32.
"""
import numpy as np

_M64 = np.uint64(0xFFFFFFFFFFFFFFFF)


def splitmix64(x):
    x = np.asarray(x, np.uint64)
    with np.errstate(over="ignore"):
        z = x + np.uint64(0x9E3779B97F4A7C15)
        z = (z ^ (z >> np.uint64(30))) * np.uint64(0xBF58476D1CE4E5B9)
        z = (z ^ (z >> np.uint64(27))) * np.uint64(0x94D049BB133111EB)
    return z ^ (z >> np.uint64(31))


def det_normal(seed, n):
    idx = np.arange(n, dtype=np.uint64)
    with np.errstate(over="ignore"):
        h = splitmix64(idx ^ splitmix64(np.uint64(seed)))
    s = np.zeros(n, np.int64)
    for k in range(4):
        s += ((h >> np.uint64(12 * k)) & np.uint64(0xFFF)).astype(np.int64)
    return ((s - 8190).astype(np.float32) / np.float32(2048.0)).astype(np.float32)


class Stream:
    """Successive det_normal blocks from one seed."""

    def __init__(self, seed):
        self.seed = seed
        self.k = 0

    def take(self, n):
        self.k += 1
        return det_normal(self.seed * 1000003 + self.k, n)


def make_cq_tensor(seed, out, inp, group, bits_, special_norms=False):
    """A synthetic CQ tensor in the archive's blob layout."""
    rng = np.random.default_rng(seed)
    in_pad = (inp + group - 1) // group * group
    rowbytes = in_pad * bits_ // 8
    packed = rng.integers(0, 256, out * rowbytes, dtype=np.uint8)
    norms = rng.uniform(0.25, 2.0, (out, in_pad // group)).astype(np.float16)
    if special_norms:
        norms.flat[::7] = np.float16(-0.75)          # negative
        norms.flat[3::11] = np.float16(3e-6)         # subnormal in fp16
        norms.flat[5::13] = np.float16(0.0)
    cb = np.concatenate([np.sort(det_normal(seed + 1, 4)), np.sort(det_normal(seed + 2, 8)),
                         np.sort(det_normal(seed + 3, 16))]).astype(np.float32)
    cb = (cb / np.sqrt(np.float32(group))).astype(np.float32)
    blob = np.concatenate([packed, norms.view(np.uint8).ravel()])
    import ndoracle as O
    return O.CQTensor(out, inp, group, bits_, blob, cb)


def make_block_weights(seed, n_layers, nh, nkv, qk, vd, d_model, group=128):
    """Per layer five synthetic 2-bit CQ tensors: q [nh*qk][d_model],
    k [nkv*qk][d_model], v [nkv*vd][d_model], gate [nh*vd][d_model],
    out_proj [d_model][nh*vd]; one shared 28-float codebook."""
    import ndoracle as O
    outs = [nh * qk, nkv * qk, nkv * vd, nh * vd, d_model]
    ins = [d_model] * 4 + [nh * vd]
    blobs = []
    cb = None
    for li in range(n_layers):
        layer = []
        for t in range(5):
            ct = make_cq_tensor(seed + 10 * li + t, outs[t], ins[t], group, 2)
            layer.append(ct.blob)
            cb = ct.codebook if cb is None else cb
        blobs.append(layer)
    return O.BlockWeights(blobs, cb, d_model, group)
