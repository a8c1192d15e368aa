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
import os
import zlib
from concurrent.futures import ThreadPoolExecutor

import numpy as np

_GOLD = np.uint64(0x9E3779B97F4A7C15)
_M1 = np.uint64(0xBF58476D1CE4E5B9)
_M2 = np.uint64(0x94D049BB133111EB)


def stream_seed(config_seed, name):
    return ((int(config_seed) << 32) ^ zlib.crc32(name.encode())) & 0xFFFFFFFFFFFFFFFF


_CHUNK = 1 << 20
# Large draws are split into 1M-element chunks computed by a thread pool (numpy's ufuncs
# release the GIL); every element is computed by the same operations in any chunking, so
# the values do not depend on the worker count.
_WORKERS = max(1, min(16, os.cpu_count() or 1))


def _chunked(n, fn):
    """fn(c0, m) for the chunks [c0, c0 + m) of range(n), in parallel when there are several."""
    spans = [(c0, min(_CHUNK, n - c0)) for c0 in range(0, n, _CHUNK)]
    if len(spans) <= 1 or _WORKERS == 1:
        for c0, m in spans:
            fn(c0, m)
        return
    with ThreadPoolExecutor(_WORKERS) as ex:
        for f in [ex.submit(fn, c0, m) for c0, m in spans]:
            f.result()


def _splitmix_into(z, seed, first):
    """z[j] = SplitMix64 output for element first + j of stream `seed`, in place."""
    t = np.empty_like(z)
    z[:] = np.arange(first + 1, first + z.size + 1, dtype=np.uint64)
    np.multiply(z, _GOLD, out=z)
    np.add(z, np.uint64(seed), out=z)
    np.right_shift(z, np.uint64(30), out=t)
    np.bitwise_xor(z, t, out=z)
    np.multiply(z, _M1, out=z)
    np.right_shift(z, np.uint64(27), out=t)
    np.bitwise_xor(z, t, out=z)
    np.multiply(z, _M2, out=z)
    np.right_shift(z, np.uint64(31), out=t)
    np.bitwise_xor(z, t, out=z)
    return z


def splitmix64(seed, n, offset=0):
    """n consecutive SplitMix64 outputs of stream `seed` starting at element `offset`."""
    out = np.empty(n, np.uint64)
    _chunked(n, lambda c0, m: _splitmix_into(out[c0:c0 + m], seed, offset + c0))
    return out


def _uniform_into(u, seed, first):
    """float64 uniforms in [0, 1) of elements first .. first + u.size - 1 of the stream."""
    z = _splitmix_into(np.empty(u.size, np.uint64), seed, first)
    np.right_shift(z, np.uint64(11), out=z)
    u[:] = z
    u *= 2.0 ** -53
    return u


def uniform(seed, n, offset=0):
    """float64 uniforms in [0, 1)."""
    u = np.empty(n, np.float64)
    _chunked(n, lambda c0, m: _uniform_into(u[c0:c0 + m], seed, offset + c0))
    return u


def _normal_flat(seed, n, mu, sigma, offset=0):
    """Normals of elements offset .. offset + n - 1 (each from uniforms 2i and 2i + 1)."""
    out = np.empty(n, np.float32)

    def one(c0, m):
        u = _uniform_into(np.empty(2 * m, np.float64), seed, 2 * (offset + c0))
        u1, u2 = u[0::2], u[1::2]
        z = np.sqrt(-2.0 * np.log1p(-u1)) * np.cos(2.0 * np.pi * u2)
        out[c0:c0 + m] = mu + sigma * z

    _chunked(n, one)
    return out


def normal_f32(config_seed, name, shape, mu=0.0, sigma=1.0):
    n = int(np.prod(shape))
    return _normal_flat(stream_seed(config_seed, name), n, mu, sigma).reshape(shape)


def uniform_f32(config_seed, name, shape, lo, hi, offset=0):
    n = int(np.prod(shape))
    u = uniform(stream_seed(config_seed, name), n, offset)
    return (lo + (hi - lo) * u).astype(np.float32).reshape(shape)


def uniform_int(config_seed, name, shape, lo, hi, dtype=np.int64, offset=0):
    """Integers uniform in [lo, hi] (inclusive), by multiply-shift of the top 32 bits."""
    n = int(np.prod(shape))
    seed = stream_seed(config_seed, name)
    out = np.empty(n, dtype)

    def one(c0, m):
        z = _splitmix_into(np.empty(m, np.uint64), seed, offset + c0)
        np.right_shift(z, np.uint64(32), out=z)
        np.multiply(z, np.uint64(hi - lo + 1), out=z)
        np.right_shift(z, np.uint64(32), out=z)
        out[c0:c0 + m] = np.int64(lo) + z.astype(np.int64)

    _chunked(n, one)
    return out.reshape(shape)


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
    n = int(np.prod(shape))
    f = _normal_flat(stream_seed(config_seed, name), n, mu, sigma)
    out = np.empty(n, np.uint16)
    _chunked(n, lambda c0, m: out.__setitem__(slice(c0, c0 + m), f32_to_bf16(f[c0:c0 + m])))
    return out.reshape(shape)


# ------------------------------------------------------------------------------------
# GGUF block tables (types.zig:113-116 Q4_0, 141-144 Q8_0)
# ------------------------------------------------------------------------------------

def f16_bits(x):
    return np.asarray(x, dtype=np.float32).astype(np.float16).view(np.uint16)


def q8_0_table(config_seed, rows, cols, name="tok_embd_q8_0"):
    """Q8_0 rows: per 32-block an f16 scale d ~ U[1e-3, 2e-2] then 32 int8 ~ U[-127, 127]."""
    nb = cols // 32
    d = f16_bits(uniform_f32(config_seed, name + ".d", (rows, nb), 1e-3, 2e-2))
    qs = uniform_int(config_seed, name + ".qs", (rows, nb, 32), -127, 127, dtype=np.int8)
    blk = np.empty((rows, nb, 34), np.uint8)
    blk[:, :, 0:2] = d.reshape(rows, nb, 1).view(np.uint8).reshape(rows, nb, 2)
    blk[:, :, 2:] = qs.view(np.uint8)
    return blk.reshape(rows, nb * 34)


def q4_0_table(config_seed, rows, cols, name="tok_embd_q4_0"):
    """Q4_0 rows: per 32-block an f16 scale d ~ U[1e-3, 2e-2] then 16 bytes of nibbles
    ~ U[0, 15] (value = nibble - 8)."""
    nb = cols // 32
    d = f16_bits(uniform_f32(config_seed, name + ".d", (rows, nb), 1e-3, 2e-2))
    qs = uniform_int(config_seed, name + ".qs", (rows, nb, 16), 0, 255, dtype=np.uint8)
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


def table_rows(kind, config_seed, ids, cols):
    """Rows `ids` of the full seeded table q8_0_table / q4_0_table / bf16_table (kind "q8_0",
    "q4_0", "bf16") of any row count, drawn straight from the streams at the rows' offsets:
    identical bytes to table(config_seed, vocab, cols)[ids] without generating the table."""
    ids = np.asarray(ids, np.int64)
    nb = cols // 32
    if kind == "bf16":
        seed = stream_seed(config_seed, "tok_embd_bf16")
        rows = [f32_to_bf16(_normal_flat(seed, cols, 0.0, 0.02, offset=int(r) * cols)) for r in ids]
        return np.stack(rows).view(np.uint8).reshape(ids.size, cols * 2)
    per, lo, hi, dt, bs = {"q8_0": (32, -127, 127, np.int8, 34), "q4_0": (16, 0, 255, np.uint8, 18)}[kind]
    name = "tok_embd_" + kind
    blk = np.empty((ids.size, nb, bs), np.uint8)
    for i, r in enumerate(ids):
        d = f16_bits(uniform_f32(config_seed, name + ".d", (nb,), 1e-3, 2e-2, offset=int(r) * nb))
        q = uniform_int(config_seed, name + ".qs", (nb, per), lo, hi, dtype=dt, offset=int(r) * nb * per)
        blk[i, :, 0:2] = d.reshape(nb, 1).view(np.uint8).reshape(nb, 2)
        blk[i, :, 2:] = q.view(np.uint8)
    return blk.reshape(ids.size, nb * bs)


def gather_ids(config_seed, n_tokens, vocab, n_repeat=64, name="ids"):
    """n_tokens ids: the first n_tokens - n_repeat uniform in [0, vocab), then n_repeat ids
    that repeat earlier ones (chosen uniformly among them)."""
    n_uni = n_tokens - n_repeat
    ids = uniform_int(config_seed, name, (n_uni,), 0, vocab - 1)
    if n_repeat > 0:
        pick = uniform_int(config_seed, name + ".rep", (n_repeat,), 0, n_uni - 1)
        ids = np.concatenate([ids, ids[pick]])
    return ids.astype(np.int32)
