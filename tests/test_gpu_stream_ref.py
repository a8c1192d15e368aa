"""hip_stream_ref, the reference streaming kernel whose fastest shape is each op's ceiling:
every launch shape (geometry x load / store form, including the global-store form) moves
exactly out_j = in0 ^ in1 (or in0) over sizes that leave a ragged last workgroup, touches
nothing past `bytes`, and works in place (out0 = in0); its copies form moves up to three
pairs of different sizes in one launch; bad arguments are refused."""
import numpy as np
import pytest

from ziglm_amd import bridge as B
from ziglm_amd import synth

pytestmark = pytest.mark.gpu

GUARD = 4096  # bytes after each buffer that must stay untouched


def _bufs(dev, nbytes, seed, n):
    """n device buffers of nbytes (+ GUARD bytes of 0x5A), filled with seeded random bytes."""
    out = []
    for i in range(n):
        host = synth.uniform_int(seed + i, "stream", (nbytes,), 0, 255).astype(np.uint8)
        b = dev.alloc(nbytes + GUARD)
        b.fill(0x5A)
        b.upload(host)
        out.append((b, host))
    return out


@pytest.mark.parametrize("nbytes", [16, 16 * 1000 + 16 * 37, 16 * (1 << 16) + 16 * 5])
@pytest.mark.parametrize("mix", [(1, 1), (2, 1), (1, 2), (2, 2)])
def test_every_shape_moves_exact_bytes(dev, nbytes, mix):
    n_in, n_out = mix
    ins = _bufs(dev, nbytes, 7, n_in)
    expect = ins[0][1] ^ ins[1][1] if n_in == 2 else ins[0][1]
    outs = _bufs(dev, nbytes, 9, n_out)
    for shape in range(dev.b.hip_stream_ref_shapes()):
        for b, _ in outs:
            b.fill(0x5A)
        dev.sync()
        rc = dev.b.hip_stream_ref(n_in, n_out, ins[0][0].ptr, ins[1][0].ptr if n_in == 2 else None,
                                  outs[0][0].ptr, outs[1][0].ptr if n_out == 2 else None, nbytes, shape,
                                  dev.stream)
        assert rc == 0, (shape, rc)
        dev.sync()
        for b, _ in outs:
            got = b.to_numpy((nbytes + GUARD,), np.uint8)
            np.testing.assert_array_equal(got[:nbytes], expect, err_msg=f"shape {shape}")
            assert np.all(got[nbytes:] == 0x5A), f"shape {shape} wrote past the end"
    for b, _ in ins + outs:
        b.deinit()


def test_in_place_form(dev):
    """out0 = in0 (the residual-stream form): in0 becomes in0 ^ in1 for every shape."""
    nbytes = 16 * 4099
    for shape in range(dev.b.hip_stream_ref_shapes()):
        (x, xh), (r, rh) = _bufs(dev, nbytes, 11, 2)
        (o1, _), = _bufs(dev, nbytes, 13, 1)
        rc = dev.b.hip_stream_ref(2, 2, x.ptr, r.ptr, x.ptr, o1.ptr, nbytes, shape, dev.stream)
        assert rc == 0
        dev.sync()
        np.testing.assert_array_equal(x.to_numpy((nbytes,), np.uint8), xh ^ rh, err_msg=f"shape {shape}")
        np.testing.assert_array_equal(o1.to_numpy((nbytes,), np.uint8), xh ^ rh, err_msg=f"shape {shape}")
        for b in (x, r, o1):
            b.deinit()


def test_refuses_bad_arguments(dev):
    a = dev.alloc(64)
    ns = dev.b.hip_stream_ref_shapes()
    assert ns == 45
    for args in ((3, 1, 64, 0), (1, 3, 64, 0), (1, 1, 24, 0), (1, 1, 64, ns), (1, 1, 64, -1)):
        n_in, n_out, nbytes, shape = args
        rc = dev.b.hip_stream_ref(n_in, n_out, a.ptr, a.ptr, a.ptr, a.ptr, nbytes, shape, dev.stream)
        assert rc == B.EINVAL, args
    # misaligned pointer
    rc = dev.b.hip_stream_ref(1, 1, a.ptr + 8, None, a.ptr, None, 32, 0, dev.stream)
    assert rc == B.EINVAL
    a.deinit()


@pytest.mark.parametrize("sizes", [(16 * 4099, 16 * 1000 + 16 * 37, 16 * 77), (16 * 5000, 0, 16 * (1 << 14) + 16 * 3),
                                   (0, 0, 16 * 33)])
@pytest.mark.parametrize("interleave", [0, 1])
def test_copies_move_exact_bytes(dev, sizes, interleave):
    """Every shape, pair by pair or interleaved, copies each pair exactly (pair 0 in place),
    leaves the bytes after each destination alone, and skips pairs of size 0 (NULL pointers
    allowed there)."""
    for shape in range(dev.b.hip_stream_ref_shapes()):
        pairs = []
        for p, nb in enumerate(sizes):
            if nb == 0:
                pairs.append((None, None, 0, None))
                continue
            (src, sh), = _bufs(dev, nb, 20 + p, 1)
            if p == 0:
                pairs.append((src, src, nb, sh))  # in place: dst = src
            else:
                (dst, _), = _bufs(dev, nb, 30 + p, 1)
                dst.fill(0x5A)
                pairs.append((src, dst, nb, sh))
        dev.sync()
        args = []
        for src, dst, nb, _ in pairs:
            args += [src.ptr if src else None, dst.ptr if dst else None, nb]
        rc = dev.b.hip_stream_ref_copies(*args, interleave, shape, dev.stream)
        assert rc == 0, (shape, rc)
        dev.sync()
        for p, (src, dst, nb, sh) in enumerate(pairs):
            if nb == 0:
                continue
            got = dst.to_numpy((nb + GUARD,), np.uint8)
            np.testing.assert_array_equal(got[:nb], sh, err_msg=f"shape {shape} pair {p}")
            assert np.all(got[nb:] == 0x5A), f"shape {shape} pair {p} wrote past the end"
        for src, dst, nb, _ in pairs:
            if nb:
                if dst is not src:
                    dst.deinit()
                src.deinit()


def test_copies_refuse_bad_arguments(dev):
    a = dev.alloc(64)
    ns = dev.b.hip_stream_ref_shapes()
    f = dev.b.hip_stream_ref_copies
    assert f(a.ptr, a.ptr, 64, None, None, 0, None, None, 0, 0, ns, dev.stream) == B.EINVAL
    assert f(a.ptr, a.ptr, 24, None, None, 0, None, None, 0, 0, 0, dev.stream) == B.EINVAL
    assert f(a.ptr, a.ptr, 64, None, None, 32, None, None, 0, 0, 0, dev.stream) == B.EINVAL  # NULL with bytes
    assert f(a.ptr + 8, a.ptr, 32, None, None, 0, None, None, 0, 0, 0, dev.stream) == B.EINVAL
    assert f(a.ptr, a.ptr, -16, None, None, 0, None, None, 0, 0, 0, dev.stream) == B.EINVAL
    assert f(None, None, 0, None, None, 0, None, None, 0, 0, 0, dev.stream) == 0  # nothing to do
    a.deinit()
