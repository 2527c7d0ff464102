"""Seeded synthetic GGUF expert weights and activations (host-side generator).

Every value is a pure function of (seed, stream, index), so any slice of a
tensor can be generated on its own, and the device generator
(k_synth_blocks / k_synth_normal in csrc/qw6_hip.hip, built on the sm_*
hash functions of csrc/qw6_dev.h) produces the same bytes:

* ``hash64(seed, stream, i)``: three SplitMix64 finalisations
  (seed key, stream key, then the counter ``i``).
* random bytes: byte ``k`` of a stream is byte ``k & 7`` of ``hash64(.., k >> 3)``.
* standard normal ``z_j``: the Irwin-Hall sum of twelve 16-bit uniforms from
  ``hash64(.., 3j .. 3j+2)``, minus 6.  Mean 0 and variance 1; computed in
  exact integer arithmetic, then divided by 65536 (exact in fp32), so no
  libm call enters and every platform reproduces it bit for bit.
* quant block ``b``: bytes from ``hash64(.., 40b + w)`` (w < 27); the fp16
  ``d`` (and ``dmin``) fields are then overwritten with
  ``fp16_rne(|z| * scale)``, z taken from ``hash64(.., 40b + 28..30)`` and
  ``(.., 40b + 31..33)``.

Block layouts follow GGUF (qw6.c:1406-1446); quant ids are qw6_quant_t
(qw6.h:76-91).
"""
from __future__ import annotations

import numpy as np

M64 = (1 << 64) - 1
GOLD = 0x9E3779B97F4A7C15
SKEY = 0xD1B54A32D192ED03
SEEDK = 0x632BE59BD9B4E019

Q_FP32, Q_Q4_K_M, Q_Q4_K_S, Q_Q5_K, Q_Q6_K = 0, 4, 5, 6, 7
Q_IQ3_S, Q_IQ2_S, Q_IQ2_XXS = 9, 11, 13

BLOCK_BYTES = {Q_Q4_K_M: 144, Q_Q4_K_S: 144, Q_Q5_K: 176, Q_Q6_K: 210,
               Q_IQ2_XXS: 66, Q_IQ2_S: 82, Q_IQ3_S: 110}
# (byte offset, |N(0,1)| multiplier) of each fp16 scale field of a block.
SCALE_FIELDS = {
    Q_Q4_K_M: ((0, 2e-3), (2, 2e-3)),
    Q_Q4_K_S: ((0, 2e-3), (2, 2e-3)),
    Q_Q5_K: ((0, 2e-3), (2, 2e-3)),
    Q_Q6_K: ((208, 1e-3),),
    Q_IQ2_XXS: ((0, 2e-3),),
    Q_IQ2_S: ((0, 1e-3),),
    Q_IQ3_S: ((0, 1e-3),),
}
HASHES_PER_BLOCK = 40

# stream kinds
K_ROUTER, K_GATE, K_UP, K_DOWN = 1, 2, 3, 4
K_SGATE, K_SUP, K_SDOWN, K_X, K_NORM, K_SROUTER = 5, 6, 7, 8, 9, 11
K_OUTPUT, K_ONORM = 12, 13   # output head: [vocab x hidden] weights, final norm


def stream_id(layer: int, kind: int, expert: int = 0) -> int:
    return (layer << 24) | (kind << 16) | expert


def _mix_int(z: int) -> int:
    z &= M64
    z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & M64
    z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & M64
    return z ^ (z >> 31)


def _mix(z: np.ndarray) -> np.ndarray:
    z = z.astype(np.uint64, copy=True)
    z ^= z >> np.uint64(30)
    z *= np.uint64(0xBF58476D1CE4E5B9)
    z ^= z >> np.uint64(27)
    z *= np.uint64(0x94D049BB133111EB)
    z ^= z >> np.uint64(31)
    return z


def stream_key(seed: int, stream: int) -> int:
    k = _mix_int(seed + SEEDK)
    return _mix_int(k ^ ((stream * SKEY) & M64))


def hash64(seed: int, stream: int, idx: np.ndarray) -> np.ndarray:
    key = np.uint64(stream_key(seed, stream))
    i = np.asarray(idx, dtype=np.uint64)
    with np.errstate(over="ignore"):
        return _mix(key + (i + np.uint64(1)) * np.uint64(GOLD))


def rand_bytes(seed: int, stream: int, n: int, start: int = 0) -> np.ndarray:
    k = np.arange(start, start + n, dtype=np.uint64)
    h = hash64(seed, stream, k >> np.uint64(3))
    return ((h >> ((k & np.uint64(7)) * np.uint64(8))) & np.uint64(0xFF)).astype(np.uint8)


def normals_from_hash(seed: int, stream: int, hidx: np.ndarray) -> np.ndarray:
    """z for the hash triples starting at hidx (exact Irwin-Hall-12)."""
    hidx = np.asarray(hidx, dtype=np.uint64)
    s = np.zeros(hidx.shape, dtype=np.int64)
    for t in range(3):
        h = hash64(seed, stream, hidx + np.uint64(t))
        for q in range(4):
            s += ((h >> np.uint64(16 * q)) & np.uint64(0xFFFF)).astype(np.int64)
    return (s - 393210).astype(np.float32) * np.float32(1.0 / 65536.0)


def normals(seed: int, stream: int, n: int, start: int = 0) -> np.ndarray:
    j = np.arange(start, start + n, dtype=np.uint64)
    return normals_from_hash(seed, stream, j * np.uint64(3))


def f32_normal(seed: int, stream: int, n: int, std: float, mean: float = 0.0) -> np.ndarray:
    z = normals(seed, stream, n) * np.float32(std)
    if mean != 0.0:
        z = np.float32(mean) + z
    return z.astype(np.float32)


def quant_blocks(seed: int, stream: int, quant: int, nblocks: int, start: int = 0) -> np.ndarray:
    """nblocks consecutive GGUF blocks (uint8 [nblocks, block_bytes])."""
    bb = BLOCK_BYTES[quant]
    b = np.arange(start, start + nblocks, dtype=np.uint64)
    j = np.arange(bb, dtype=np.uint64)
    hidx = b[:, None] * np.uint64(HASHES_PER_BLOCK) + (j[None, :] >> np.uint64(3))
    h = hash64(seed, stream, hidx)
    out = ((h >> ((j[None, :] & np.uint64(7)) * np.uint64(8))) & np.uint64(0xFF)).astype(np.uint8)
    for f, (off, scale) in enumerate(SCALE_FIELDS[quant]):
        z = normals_from_hash(seed, stream, b * np.uint64(HASHES_PER_BLOCK) + np.uint64(28 + 3 * f))
        half = (np.abs(z) * np.float32(scale)).astype(np.float32).astype(np.float16)
        hv = half.view(np.uint16)
        out[:, off] = (hv & 0xFF).astype(np.uint8)
        out[:, off + 1] = (hv >> 8).astype(np.uint8)
    return out


def row_bytes(quant: int, cols: int) -> int:
    if quant == Q_FP32:
        return cols * 4
    assert cols % 256 == 0
    return cols // 256 * BLOCK_BYTES[quant]


def quant_matrix(seed: int, stream: int, quant: int, rows: int, cols: int) -> np.ndarray:
    """A rows x cols GGUF matrix as a flat uint8 array (rows consecutive)."""
    nb = rows * (cols // 256)
    return quant_blocks(seed, stream, quant, nb).reshape(-1)


def zipf_logits(seed: int, tokens: int, n_experts: int = 256, s: float = 1.1) -> np.ndarray:
    """Router logits whose softmax top-k is a Zipf(s)-weighted draw without
    replacement (Gumbel-top-k): logit[t, e] = ln z_pi(e) + Gumbel(0, 1), with
    z_r = r^-s and pi a seeded permutation of the experts."""
    rank = np.argsort(rand_bytes(seed, stream_id(0, 12), 4 * n_experts)
                      .view(np.uint32)[:n_experts], kind="stable")
    logz = -s * np.log(np.arange(1, n_experts + 1, dtype=np.float64))
    base = np.empty(n_experts, dtype=np.float64)
    base[rank] = logz
    u = (hash64(seed, stream_id(0, 13), np.arange(tokens * n_experts, dtype=np.uint64))
         >> np.uint64(11)).astype(np.float64) * (1.0 / (1 << 53))
    u = np.clip(u, 1e-300, 1.0 - 1e-16)
    g = -np.log(-np.log(u))
    return (base[None, :] + g.reshape(tokens, n_experts)).astype(np.float32)
