"""GPU parity of the linear projections (streaming/linear.rs:269-576) through
the C ABI, against the CPU oracle (ops.rs:62-105 arithmetic).

- The reference's own known-answer tests (streaming/tests.rs:2078-2181,
  ops.rs:488-495) run through the GPU.
- The q/k/v/o projection shapes of the BASELINE models, bf16 weights, at
  decode (batch 1 and 4: GEMV kernel) and prefill batches (16, 300, 4096:
  MFMA kernel with split activations): max |gpu - oracle| <= 1e-4 x max |oracle|
  (the f32 bar of the attention path; observed errors are about 1e-6).
- The generic kernel (other dtypes at large batch, odd in_features) sums in
  the oracle's order and must match it bit for bit.
"""
import zlib

import numpy as np
import pytest

import oracle as o
import spissa_amd as sa
from spissa_amd.linear import (DTYPE_BF16, DTYPE_F16, DTYPE_F32, MissingTensorError,
                               StreamingLinearConfig, StreamingTileLinearConfig)
from spissa_amd.synth import normal_f32, seed_for
from tests.helpers import assert_bitwise, rel_err

pytestmark = pytest.mark.gpu

TOL = 1e-4

# (model, hidden, q_out, kv_out) of the BASELINE configs
MODELS = {
    "llama32_1b": (2048, 2048, 512),
    "llama32_3b": (3072, 3072, 1024),
    "gemma3_1b": (1152, 1024, 256),
    "gemma3_4b": (2560, 2048, 1024),
}


def seed(a: int, b: int, c, tag: str) -> int:
    """A distinct generator seed per (a, b, c, tag)."""
    return seed_for(90 + a, b, int(c), "q", zlib.crc32(tag.encode()))


def bf16_bits(x: np.ndarray) -> np.ndarray:
    b = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    return ((b + 0x7FFF + ((b >> 16) & 1)) >> 16).astype(np.uint16)


def weight(out_f, in_f, dtype, tag):
    wf = normal_f32(seed(0, out_f, in_f, tag), out_f * in_f, 0.0, 0.02)
    if dtype == DTYPE_F32:
        return wf
    if dtype == DTYPE_F16:
        return wf.astype(np.float16).view(np.uint16).copy()
    return bf16_bits(wf)


def acts(batch, in_f, tag):
    return normal_f32(seed(1, batch, in_f, tag), batch * in_f)


def check_close(got, ref, what):
    err = rel_err(got, ref)
    print(f"[linear] {what}: rel err {err:.2e}", flush=True)
    assert err <= TOL, f"{what}: rel err {err}"


@pytest.mark.parametrize("dtype,bits", [(DTYPE_F16, [0x3800, 0xBC00, 0x4000, 0xC000, 0x3400, 0x3800,
                                                     0x3C00, 0x3C00, 0xBC00, 0x0000, 0xB800, 0x3A00]),
                                        (DTYPE_BF16, [0x3F00, 0xBF80, 0x4000, 0xC000, 0x3E80, 0x3F00,
                                                      0x3F80, 0x3F80, 0xBF80, 0x0000, 0xBF00, 0x3F40])])
def test_raw_16bit_batch1_linear_kat_on_gpu(gpu, dtype, bits):
    # streaming/tests.rs:2078-2181: exact values, 1e-6 in the reference
    model = sa.LinearModel({"w": sa.LinearWeight(np.array(bits, np.uint16), dtype, 4, 3)})
    out = sa.streaming_tile_linear_from_model(
        model, "w", np.array([1.5, -2.0, 0.25], np.float32), np.array([0.0, 0.5, -1.0, 4.0], np.float32),
        StreamingTileLinearConfig(StreamingLinearConfig(1, 3, 4), 2))
    assert out.tolist() == [3.25, -2.875, -1.75, 5.1875]


def test_linear_uses_transposed_weight_layout_on_gpu(gpu):
    # ops.rs:488-495
    w = sa.LinearWeight(np.array([1, 0, 1, 0.5, 0.5, 0.5], np.float32), DTYPE_F32, 2, 3)
    out = sa.linear(w, np.array([1, 2, 3], np.float32), np.array([1, -1], np.float32),
                    StreamingLinearConfig(1, 3, 2))
    assert out.tolist() == [5.0, 2.0]


@pytest.mark.parametrize("model", list(MODELS))
@pytest.mark.parametrize("batch", [1, 4, 16, 300])
def test_bf16_projections_match_oracle(gpu, model, batch):
    hidden, q_out, kv_out = MODELS[model]
    for name, (out_f, in_f) in {"q": (q_out, hidden), "kv": (kv_out, hidden), "o": (hidden, q_out)}.items():
        w = weight(out_f, in_f, DTYPE_BF16, f"{model}.{name}")
        x = acts(batch, in_f, f"{model}.{name}")
        bias = normal_f32(seed(2, out_f, 0, name), out_f) if name == "kv" else None
        lw = sa.LinearWeight(w, DTYPE_BF16, out_f, in_f)
        got = sa.linear(lw, x, bias, StreamingLinearConfig(batch, in_f, out_f))
        rows = min(batch, 16)
        pick = np.unique(np.linspace(0, batch - 1, rows).astype(int))
        xs = x.reshape(batch, in_f)[pick].ravel().copy()
        ref = o.linear(xs, w, o.DTYPE_BF16, bias, len(pick), in_f, out_f)
        check_close(got.reshape(batch, out_f)[pick].ravel(), ref, f"{model} {name} batch {batch}")


def test_llama3b_fused_qkv_prefill_4096(gpu):
    # the prefill projection at full size: [4096, 3072] x [5120, 3072]^T
    hidden, out_f, batch = 3072, 5120, 4096
    w = weight(out_f, hidden, DTYPE_BF16, "qkv")
    x = acts(batch, hidden, "qkv")
    got = sa.linear(sa.LinearWeight(w, DTYPE_BF16, out_f, hidden), x, None,
                    StreamingLinearConfig(batch, hidden, out_f))
    pick = np.array([0, 1, 127, 128, 1000, 2047, 2048, 3333, 4094, 4095])
    ref = o.linear(x.reshape(batch, hidden)[pick].ravel().copy(), w, o.DTYPE_BF16, None, len(pick), hidden,
                   out_f)
    check_close(got.reshape(batch, out_f)[pick].ravel(), ref, "llama3b qkv prefill 4096")
    assert np.isfinite(got).all()


def test_wide_tile_gemm_ragged_edges(gpu):
    # 4000 x 5100 outputs take the 256 x 320 tiles (one round of 256; 128 x 256
    # tiles would need 640 workgroups): the last row and column tiles are
    # partial, and K = 96 is an odd number of 32-deep k tiles.
    batch, in_f, out_f = 4000, 96, 5100
    w = weight(out_f, in_f, DTYPE_BF16, "wide")
    x = acts(batch, in_f, "wide")
    bias = normal_f32(seed(5, out_f, in_f, "b"), out_f)
    got = sa.linear(sa.LinearWeight(w, DTYPE_BF16, out_f, in_f), x, bias,
                    StreamingLinearConfig(batch, in_f, out_f))
    pick = np.array([0, 1, 255, 256, 1777, 3839, 3840, 3998, 3999])
    ref = o.linear(x.reshape(batch, in_f)[pick].ravel().copy(), w, o.DTYPE_BF16, bias, len(pick), in_f, out_f)
    check_close(got.reshape(batch, out_f)[pick].ravel(), ref, "wide tiles 4000 x 5100 x 96")
    assert np.isfinite(got).all()


@pytest.mark.parametrize("dtype", [DTYPE_F16, DTYPE_F32])
@pytest.mark.parametrize("batch", [1, 3])
def test_f16_f32_weights_gemv(gpu, dtype, batch):
    out_f, in_f = 1024, 3072
    w = weight(out_f, in_f, dtype, "gemv")
    x = acts(batch, in_f, "gemv")
    bias = normal_f32(seed(3, out_f, dtype, "b"), out_f)
    got = sa.linear(sa.LinearWeight(w, dtype, out_f, in_f), x, bias, StreamingLinearConfig(batch, in_f, out_f))
    ref = o.linear(x, w, dtype, bias, batch, in_f, out_f)
    check_close(got, ref, f"dtype {dtype} batch {batch}")


@pytest.mark.parametrize("dtype,batch,in_f,out_f", [
    (DTYPE_F32, 8, 256, 100),    # f32 weights beyond the GEMV batch
    (DTYPE_F16, 6, 96, 70),
    (DTYPE_BF16, 8, 100, 33),    # in_features not a multiple of 32
    (DTYPE_BF16, 1, 13, 7),      # in_features not a multiple of 8
])
def test_generic_path_is_bitwise_the_oracle(gpu, dtype, batch, in_f, out_f):
    w = weight(out_f, in_f, dtype, "generic")
    x = acts(batch, in_f, "generic")
    bias = normal_f32(seed(4, out_f, in_f, "b"), out_f)
    got = sa.linear(sa.LinearWeight(w, dtype, out_f, in_f), x, bias, StreamingLinearConfig(batch, in_f, out_f))
    assert_bitwise(got, o.linear(x, w, dtype, bias, batch, in_f, out_f), "generic linear")


def test_ragged_gemm_tiles(gpu):
    # batch and out_features not multiples of the 128 x 128 tile; no bias
    batch, in_f, out_f = 130, 64, 200
    w = weight(out_f, in_f, DTYPE_BF16, "ragged")
    x = acts(batch, in_f, "ragged")
    got = sa.linear(sa.LinearWeight(w, DTYPE_BF16, out_f, in_f), x, None, StreamingLinearConfig(batch, in_f, out_f))
    check_close(got, o.linear(x, w, o.DTYPE_BF16, None, batch, in_f, out_f), "ragged 130x200")


def test_device_tier_matches_dropin(gpu):
    import torch

    from spissa_amd.device import Session

    batch, in_f, out_f = 64, 2048, 512
    w = weight(out_f, in_f, DTYPE_BF16, "dev")
    x = acts(batch, in_f, "dev")
    bias = normal_f32(seed(5, out_f, 0, "b"), out_f)
    st = torch.cuda.Stream()
    s = Session(0, stream=st)
    lw = s.linear_weight(w, DTYPE_BF16, out_f, in_f)
    with torch.cuda.stream(st):
        dx = torch.from_numpy(x).cuda()
        db = torch.from_numpy(bias).cuda()
        dout = torch.empty(batch * out_f, device="cuda")
        s.linear(lw, dx, db, batch, dout)
    s.sync()
    ref = sa.linear(sa.LinearWeight(w, DTYPE_BF16, out_f, in_f), x, bias, StreamingLinearConfig(batch, in_f, out_f))
    assert_bitwise(dout.cpu().numpy(), ref, "device tier vs drop-in")


def test_linear_errors(gpu):
    w = sa.LinearWeight(np.zeros(6, np.float32), DTYPE_F32, 2, 3)
    x = np.ones(3, np.float32)
    with pytest.raises(sa.ShapeError):  # input len
        sa.linear(w, np.ones(4, np.float32), None, StreamingLinearConfig(1, 3, 2))
    with pytest.raises(sa.ShapeError):  # bias len
        sa.linear(w, x, np.ones(3, np.float32), StreamingLinearConfig(1, 3, 2))
    with pytest.raises(sa.ShapeError):  # weight shape vs config
        sa.linear(w, np.ones(2, np.float32), None, StreamingLinearConfig(1, 2, 3))
    with pytest.raises(sa.InvalidTensorDataError):  # stored bytes vs shape x dtype
        sa.LinearWeight(np.zeros(5, np.float32), DTYPE_F32, 2, 3)
    model = sa.LinearModel({"w": w})
    with pytest.raises(MissingTensorError):
        sa.streaming_tile_linear_from_model(model, "nope", x, None,
                                            StreamingTileLinearConfig(StreamingLinearConfig(1, 3, 2), 4))
    with pytest.raises(sa.ShapeError):  # streaming/validation.rs:249-256
        sa.streaming_tile_linear_from_model(model, "w", x, None,
                                            StreamingTileLinearConfig(StreamingLinearConfig(1, 3, 2), 0))
    out = sa.linear(w, np.zeros(0, np.float32), None, StreamingLinearConfig(0, 3, 2))
    assert out.size == 0
