"""Empty inputs through the C-ABI: every fused op, gather, product and attention call with zero
rows / tokens / elements is a no-op that reports no error (the strict device wrapper raises
on any) and leaves every output byte as it was."""
import numpy as np
import pytest

from ziglm_amd import bridge as B

pytestmark = pytest.mark.gpu

H, D, NH, NKV = 256, 128, 4, 2
SIZE = 1 << 16


@pytest.fixture
def bufs(dev):
    names = ("x", "r", "out", "w1", "w2", "q", "k", "v", "kc", "vc", "pos", "tab", "ids", "y", "ws")
    b = {n: dev.alloc(SIZE) for n in names}
    for v in b.values():
        v.fill(0x5A)
    dev.sync()
    yield b
    for v in b.values():
        v.deinit()


def untouched(dev, b):
    dev.sync()
    for name, v in b.items():
        assert np.all(v.to_numpy((SIZE,), np.uint8) == 0x5A), name


@pytest.mark.parametrize("dtype", [B.F32, B.BF16])
def test_row_ops_with_zero_rows(dev, bufs, dtype):
    b = bufs
    dev.rmsNormRows(dtype, b["x"], b["w1"], b["out"], 0, H, 1e-6, 1)
    dev.addRmsNormRows(dtype, b["x"], b["r"], b["w1"], b["out"], 0, H, 1e-6, 1)
    dev.rmsnormAddRows(dtype, b["x"], b["r"], b["w1"], 0, H, 1e-6, 1)
    dev.rmsNormAddRmsNorm(dtype, b["x"], b["r"], b["w1"], b["w2"], b["out"], 0, H, 1e-6, 1)
    dev.gegluEx(dtype, b["x"], b["r"], b["out"], 0)
    dev.tanhSoftcapEx(dtype, b["x"], 30.0, 0)
    untouched(dev, b)


def test_reference_abi_ops_with_zero_elements(dev, bufs):
    b = bufs
    dev.rmsNorm(b["x"], b["w1"], b["out"], 0, 1e-6, 1)
    dev.addRmsNorm(b["x"], b["r"], b["w1"], b["out"], 0, 1e-6, 1)
    dev.rmsnormAdd(b["x"], b["r"], b["w1"], 0, 1e-6, 1)
    dev.geglu(b["x"], b["r"], b["out"], 0)
    dev.tanhSoftcap(b["x"], 30.0, 0)
    dev.add(b["x"], b["r"], 0)
    untouched(dev, b)


@pytest.mark.parametrize("dtype", [B.F32, B.BF16])
def test_qk_norm_rope_kv_with_zero_tokens(dev, bufs, dtype):
    b = bufs
    dev.qkNormRopeKv(dtype, b["q"], b["k"], b["v"], b["w1"], b["w2"], 0, b["kc"], b["vc"], 16, 0, 16,
                     NKV * D, b["pos"], 0, None, 0, NH, NKV, D, 0, 10000.0, 1.0, 1e-6, 1)
    untouched(dev, b)


@pytest.mark.parametrize("qtype", [B.Q8_0, B.Q4_0, B.BF16, B.F32])
@pytest.mark.parametrize("out_dtype", [B.F32, B.BF16])
def test_gather_with_zero_tokens(dev, bufs, qtype, out_dtype):
    b = bufs
    dev.embedGather(b["tab"], qtype, 4, b["ids"], out_dtype, b["out"], 0, H, 16.0)
    untouched(dev, b)


@pytest.mark.parametrize("qtype", [B.Q4_0, B.Q8_0, B.BF16, B.F32])
def test_products_with_zero_tokens(dev, bufs, qtype):
    b = bufs
    dev.gemm(qtype, b["w1"], b["x"], b["y"], 0, 64, H)
    dev.gemmEx(qtype, b["w1"], None, B.BF16, b["x"], B.BF16, b["y"], 0, 64, H)
    untouched(dev, b)


def test_attention_with_zero_sequences(dev, bufs):
    b = bufs
    dev.attentionDecode(B.F32, b["q"], b["kc"], b["vc"], b["out"], 16, NKV * D, None, 0, b["pos"], 0, 16, 0,
                        NH, NKV, D, 1.0, 0.0, 0, b["ws"], SIZE)
    untouched(dev, b)
