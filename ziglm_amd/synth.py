"""Seeded synthetic inputs for the fused per-layer ops, one documented generator.

Generator: counter-based SplitMix64. Stream s, element i:
    z = s + (i + 1) * 0x9E3779B97F4A7C15  (mod 2^64), then the SplitMix64 finaliser
    z ^= z >> 30; z *= 0xBF58476D1CE4E5B9; z ^= z >> 27; z *= 0x94D049BB133111EB; z ^= z >> 31
Uniform doubles use the top 53 bits: u = (z >> 11) * 2^-53 in [0, 1).
Normals use Box-Muller on two independent uniform draws (elements 2i and 2i+1 of the
stream): n = sqrt(-2 ln(1 - u1)) * cos(2 pi u2), computed in float64, then scaled
(mu + sigma*n) and rounded to f32 (round to nearest even); bf16 tensors are the f32 value
rounded with ziglm's quant.f32ToBf16 (quant.zig:35-40).
Stream seeds: s = (config_seed << 32) ^ crc32(tensor_name), so each tensor of a config has
its own stream and the values do not depend on which other tensors are drawn.

The reference names seeds but not a generator (its Zig DefaultPrng cannot run here), so
this generator is the fixed convention for every config in BASELINE.json.
"""
import zlib

import numpy as np

_GOLD = np.uint64(0x9E3779B97F4A7C15)
_M1 = np.uint64(0xBF58476D1CE4E5B9)
_M2 = np.uint64(0x94D049BB133111EB)


def stream_seed(config_seed, name):
    return ((int(config_seed) << 32) ^ zlib.crc32(name.encode())) & 0xFFFFFFFFFFFFFFFF


_CHUNK = 1 << 20


def splitmix64(seed, n, offset=0):
    """n consecutive SplitMix64 outputs of stream `seed` starting at element `offset`.
    Computed in place over 1M-element chunks (fresh large arrays are slow to fault in)."""
    out = np.empty(n, np.uint64)
    tmp = np.empty(min(n, _CHUNK), np.uint64)
    s = np.uint64(seed)
    for c0 in range(0, n, _CHUNK):
        m = min(_CHUNK, n - c0)
        z, t = out[c0:c0 + m], tmp[:m]
        z[:] = np.arange(offset + c0 + 1, offset + c0 + m + 1, dtype=np.uint64)
        np.multiply(z, _GOLD, out=z)
        np.add(z, s, out=z)
        np.right_shift(z, np.uint64(30), out=t)
        np.bitwise_xor(z, t, out=z)
        np.multiply(z, _M1, out=z)
        np.right_shift(z, np.uint64(27), out=t)
        np.bitwise_xor(z, t, out=z)
        np.multiply(z, _M2, out=z)
        np.right_shift(z, np.uint64(31), out=t)
        np.bitwise_xor(z, t, out=z)
    return out


def uniform(seed, n):
    """float64 uniforms in [0, 1)."""
    z = splitmix64(seed, n)
    np.right_shift(z, np.uint64(11), out=z)
    u = z.astype(np.float64)
    u *= 2.0 ** -53
    return u


def normal_f32(config_seed, name, shape, mu=0.0, sigma=1.0):
    n = int(np.prod(shape))
    u = uniform(stream_seed(config_seed, name), 2 * n)
    out = np.empty(n, np.float32)
    for c0 in range(0, n, _CHUNK):
        m = min(_CHUNK, n - c0)
        u1 = u[2 * c0:2 * (c0 + m):2]
        u2 = u[2 * c0 + 1:2 * (c0 + m):2]
        z = np.sqrt(-2.0 * np.log1p(-u1)) * np.cos(2.0 * np.pi * u2)
        out[c0:c0 + m] = mu + sigma * z
    return out.reshape(shape)


def uniform_f32(config_seed, name, shape, lo, hi):
    n = int(np.prod(shape))
    u = uniform(stream_seed(config_seed, name), n)
    return (lo + (hi - lo) * u).astype(np.float32).reshape(shape)


def uniform_int(config_seed, name, shape, lo, hi):
    """Integers uniform in [lo, hi] (inclusive), by multiply-shift of the top 32 bits."""
    n = int(np.prod(shape))
    z = splitmix64(stream_seed(config_seed, name), n)
    np.right_shift(z, np.uint64(32), out=z)
    np.multiply(z, np.uint64(hi - lo + 1), out=z)
    np.right_shift(z, np.uint64(32), out=z)
    return (np.int64(lo) + z.astype(np.int64)).reshape(shape)


def f32_to_bf16(x):
    """ziglm quant.f32ToBf16 (quant.zig:35-40): (bits + 0x7FFF + lsb) >> 16, NaN not
    special-cased."""
    b = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    r = (b + np.uint64(0x7FFF) + ((b >> np.uint64(16)) & np.uint64(1))) >> np.uint64(16)
    return (r & np.uint64(0xFFFF)).astype(np.uint16)


def bf16_to_f32(u):
    """ziglm quant.bf16ToF32 (quant.zig:30-33)."""
    return (np.ascontiguousarray(u, dtype=np.uint16).astype(np.uint32) << np.uint32(16)).view(np.float32)


def normal_bf16(config_seed, name, shape, mu=0.0, sigma=1.0):
    return f32_to_bf16(normal_f32(config_seed, name, shape, mu, sigma))


# ------------------------------------------------------------------------------------
# GGUF block tables (types.zig:113-116 Q4_0, 141-144 Q8_0)
# ------------------------------------------------------------------------------------

def f16_bits(x):
    return np.asarray(x, dtype=np.float32).astype(np.float16).view(np.uint16)


def q8_0_table(config_seed, rows, cols, name="tok_embd_q8_0"):
    """Q8_0 rows: per 32-block an f16 scale d ~ U[1e-3, 2e-2] then 32 int8 ~ U[-127, 127]."""
    nb = cols // 32
    d = f16_bits(uniform_f32(config_seed, name + ".d", (rows, nb), 1e-3, 2e-2))
    qs = uniform_int(config_seed, name + ".qs", (rows, nb, 32), -127, 127).astype(np.int8)
    blk = np.empty((rows, nb, 34), np.uint8)
    blk[:, :, 0:2] = d.reshape(rows, nb, 1).view(np.uint8).reshape(rows, nb, 2)
    blk[:, :, 2:] = qs.view(np.uint8)
    return blk.reshape(rows, nb * 34)


def q4_0_table(config_seed, rows, cols, name="tok_embd_q4_0"):
    """Q4_0 rows: per 32-block an f16 scale d ~ U[1e-3, 2e-2] then 16 bytes of nibbles
    ~ U[0, 15] (value = nibble - 8)."""
    nb = cols // 32
    d = f16_bits(uniform_f32(config_seed, name + ".d", (rows, nb), 1e-3, 2e-2))
    qs = uniform_int(config_seed, name + ".qs", (rows, nb, 16), 0, 255).astype(np.uint8)
    blk = np.empty((rows, nb, 18), np.uint8)
    blk[:, :, 0:2] = d.reshape(rows, nb, 1).view(np.uint8).reshape(rows, nb, 2)
    blk[:, :, 2:] = qs
    return blk.reshape(rows, nb * 18)


def q6_k_table(config_seed, rows, cols, name="q6k"):
    """Q6_K rows (types.zig:187-192): per 256-super-block random ql / qh / int8 scales and an
    f16 d ~ U[1e-3, 2e-2]."""
    nsb = cols // 256
    raw = uniform_int(config_seed, name, (rows, nsb, 210), 0, 255).astype(np.uint8)
    d = f16_bits(uniform_f32(config_seed, name + ".d", (rows, nsb), 1e-3, 2e-2))
    raw[:, :, 208:210] = d.reshape(rows, nsb, 1).view(np.uint8).reshape(rows, nsb, 2)
    return raw.reshape(rows, nsb * 210)


def q4_k_table(config_seed, rows, cols, name="q4k"):
    """Q4_K rows (types.zig:170-175): per 256-super-block f16 d ~ U[1e-3, 2e-2], f16 dmin ~
    U[1e-3, 1e-2], random packed 6-bit scales / mins and nibbles."""
    nsb = cols // 256
    raw = uniform_int(config_seed, name, (rows, nsb, 144), 0, 255).astype(np.uint8)
    d = f16_bits(uniform_f32(config_seed, name + ".d", (rows, nsb), 1e-3, 2e-2))
    m = f16_bits(uniform_f32(config_seed, name + ".dmin", (rows, nsb), 1e-3, 1e-2))
    raw[:, :, 0:2] = d.reshape(rows, nsb, 1).view(np.uint8).reshape(rows, nsb, 2)
    raw[:, :, 2:4] = m.reshape(rows, nsb, 1).view(np.uint8).reshape(rows, nsb, 2)
    return raw.reshape(rows, nsb * 144)


def bf16_table(config_seed, rows, cols, name="tok_embd_bf16"):
    """BF16 rows ~ N(0, 0.02), as little-endian bytes."""
    return normal_bf16(config_seed, name, (rows, cols), 0.0, 0.02).view(np.uint8).reshape(rows, cols * 2)


def gather_ids(config_seed, n_tokens, vocab, n_repeat=64, name="ids"):
    """n_tokens ids: the first n_tokens - n_repeat uniform in [0, vocab), then n_repeat ids
    that repeat earlier ones (chosen uniformly among them)."""
    n_uni = n_tokens - n_repeat
    ids = uniform_int(config_seed, name, (n_uni,), 0, vocab - 1)
    if n_repeat > 0:
        pick = uniform_int(config_seed, name + ".rep", (n_repeat,), 0, n_uni - 1)
        ids = np.concatenate([ids, ids[pick]])
    return ids.astype(np.int32)
