"""Host restatement of the library's random streams, for the tests: Philox4x32-10 (Salmon, Moraes,
Dror, Shaw, "Parallel random numbers: as easy as 1, 2, 3", SC'11), its (0, 1) uniform mapping, the
Box-Muller pair of the action noise and the U(-1, 1) draws of the resets.

The library keys Philox with the env's 64-bit seed (low word k0, high word k1) and draws with the
counter (world, per-world control-step counter, stream, index):
* action noise of control step t: stream 0, index = action pair p (actions 2p and 2p + 1 take the
  cosine and sine normals of one draw);
* auto-reset noise of a world that finishes step t: stream 1, index = actuated joint;
* g1_env_reset noise: stream 2, index = actuated joint.
The counter is 0 at env creation and grows by one per g1_env_reset and per control step.

Replaces the reference's curand XORWOW streams (src/g1_env.cu:94,105,206,310), which come from a
closed library and cannot be reproduced. The words are pinned by the Random123 known-answer vectors
(tests/test_noise_host.py); the float mappings are restated here in float32 numpy arithmetic, which
rounds like the kernel's.
"""
import numpy as np

M0, M1 = np.uint64(0xD2511F53), np.uint64(0xCD9E8D57)
W0, W1 = np.uint32(0x9E3779B9), np.uint32(0xBB67AE85)
STREAM_ACTION, STREAM_RESET, STREAM_INIT = 0, 1, 2


def philox4x32_10(ctr, k0, k1):
    """ctr: uint32 [..., 4]; returns the four output words, uint32 [..., 4]."""
    c = np.asarray(ctr, np.uint32)
    x, y, z, w = (c[..., i].astype(np.uint64) for i in range(4))
    k0, k1 = np.uint32(k0), np.uint32(k1)
    mask = np.uint64(0xFFFFFFFF)
    for _ in range(10):
        p0, p1 = M0 * x, M1 * z
        hi0, lo0 = p0 >> np.uint64(32), p0 & mask
        hi1, lo1 = p1 >> np.uint64(32), p1 & mask
        x, y, z, w = hi1 ^ y ^ np.uint64(k0), lo1, hi0 ^ w ^ np.uint64(k1), lo0
        k0 = np.uint32((int(k0) + int(W0)) & 0xFFFFFFFF)
        k1 = np.uint32((int(k1) + int(W1)) & 0xFFFFFFFF)
    return np.stack([x, y, z, w], -1).astype(np.uint32)


def u01(v):
    """The 24 high bits of a word plus one half, scaled by 2^-24, in float32: in (0, 1], never 0
    (the top 2^23 values round to even, so the largest word gives exactly 1)."""
    hi = (np.asarray(v, np.uint32) >> np.uint32(8)).astype(np.float32)
    return (hi + np.float32(0.5)) * np.float32(1.0 / 16777216.0)


def _words(seed, worlds, step, stream, index):
    worlds = np.asarray(worlds, np.uint32)
    step = np.broadcast_to(np.asarray(step, np.uint32), worlds.shape)
    idx = np.asarray(index, np.uint32)
    c = np.zeros(worlds.shape + idx.shape + (4,), np.uint32)
    c[..., 0] = worlds[..., None]
    c[..., 1] = step[..., None]
    c[..., 2] = stream
    c[..., 3] = idx
    return philox4x32_10(c, seed & 0xFFFFFFFF, (seed >> 32) & 0xFFFFFFFF)


def action_noise(seed, worlds, step, nact=29):
    """Standard normals of the action noise, float32 [len(worlds), nact]: pair p's draw gives
    sqrt(-2 ln u1) cos(theta) to action 2p and sqrt(-2 ln u1) sin(theta) to 2p + 1, with u1, u2
    the uniforms of its first two words and theta the float32 product 2 pi u2. Evaluated in
    float64 and rounded once: the kernel's float32 log, square root and sincos differ from it by a
    few ulp."""
    r = _words(seed, worlds, step, STREAM_ACTION, np.arange((nact + 1) // 2))
    u1, u2 = u01(r[..., 0]), u01(r[..., 1])
    theta = (np.float32(6.2831853071795864) * u2).astype(np.float64)
    rad = np.sqrt(-2.0 * np.log(u1.astype(np.float64)))
    z = np.stack([rad * np.cos(theta), rad * np.sin(theta)], -1).reshape(len(np.atleast_1d(worlds)), -1)
    return z[:, :nact].astype(np.float32)


def uniform_pm1(seed, worlds, step, stream, nact=29):
    """U(-1, 1) draws of a reset stream, float32 [len(worlds), nact]: 2 u01(word 0) - 1 in float32,
    bit for bit the kernel's value."""
    r = _words(seed, worlds, step, stream, np.arange(nact))
    return u01(r[..., 0]) * np.float32(2.0) - np.float32(1.0)
