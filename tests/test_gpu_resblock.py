"""The fused stride-1 identity BasicBlock (vdk_resblock3x3) through the C ABI.

One BasicBlock of the ResNet trunk (src/encoder_resnet.cpp:33-48) is
y = relu(conv2(relu(conv1(x) + b1)) + b2 + x).  The fused launch keeps the
intermediate map in LDS; its arithmetic is the halo conv kernel's, so it must
equal the same block run as two vdk_conv2d_nhwc launches bit for bit, and it is
checked against the oracle's f32 convs (intermediate rounded to f16, as both GPU
paths store it) at the per-layer conv tolerance.
"""
import zlib

import numpy as np
import pytest

import pyoracle as O
from gpu_util import announce, close_report, conv_gpu, device_ok
from vdamd import lib

pytestmark = [pytest.mark.gpu, pytest.mark.skipif(not device_ok(), reason="no HIP device")]

HALO_TILE = 28        # the 32-channel halo conv tile the fused kernel matches
CONV_RTOL = 2e-3
CONV_ATOL_RMS = 2e-3


def _block_params(rng, C):
    w1 = (rng.standard_normal((C, C, 3, 3), dtype=np.float32) * np.sqrt(2.0 / (9 * C))).astype(np.float16)
    w2 = (rng.standard_normal((C, C, 3, 3), dtype=np.float32) * np.sqrt(2.0 / (9 * C))).astype(np.float16)
    b1 = (rng.standard_normal(C, dtype=np.float32) * 0.1).astype(np.float32)
    b2 = (rng.standard_normal(C, dtype=np.float32) * 0.1).astype(np.float32)
    return w1, b1, w2, b2


def _pack(w):
    return np.ascontiguousarray(w.transpose(0, 2, 3, 1))   # [OC][KH][KW][IC]


def resblock_gpu(x, w1, b1, w2, b2, variant=-1):
    L = lib.lib()
    x = np.ascontiguousarray(x, dtype=np.float16)
    B, H, W, C = x.shape
    dx = lib.DeviceBuffer.from_array(x)
    dw1, dw2 = lib.DeviceBuffer.from_array(_pack(w1)), lib.DeviceBuffer.from_array(_pack(w2))
    db1, db2 = lib.DeviceBuffer.from_array(b1), lib.DeviceBuffer.from_array(b2)
    dy = lib.DeviceBuffer(x.nbytes)
    lib.check(L.vdk_resblock3x3_variant(dx.ptr, B, H, W, C, dw1.ptr, db1.ptr, dw2.ptr, db2.ptr, dy.ptr,
                                        variant, None))
    lib.check(L.vdk_synchronize())
    return dy.to_array(np.float16, x.shape)


def two_launch_block(x, w1, b1, w2, b2):
    t = conv_gpu(x, w1, b1, None, 1, 1, relu=True, tile=HALO_TILE)
    return conv_gpu(t, w2, b2, x, 1, 1, relu=True, tile=HALO_TILE)


CASES = [
    # (B, H, W): the ResNet34 stage-1 map (80 mel x 298 frames), tiles cut
    # in both directions, exact tile multiples, a single pixel, one row
    (2, 80, 298),
    (3, 5, 7),
    (1, 13, 61),
    (1, 12, 60),
    (2, 1, 1),
    (1, 1, 97),
    (2, 33, 2),
]


@pytest.mark.parametrize("variant", [-1, 1, 2])
@pytest.mark.parametrize("case", CASES, ids=[f"{b}x{h}x{w}" for b, h, w in CASES])
def test_resblock_equals_two_launches(case, variant):
    B, H, W = case
    C = 32
    rng = np.random.default_rng(zlib.crc32(f"rb{B}x{H}x{W}".encode()))
    x = np.maximum(rng.standard_normal((B, H, W, C), dtype=np.float32), 0).astype(np.float16)
    w1, b1, w2, b2 = _block_params(rng, C)
    announce(f"resblock3x3 B={B} H={H} W={W} C={C} variant={variant}")
    got = resblock_gpu(x, w1, b1, w2, b2, variant)
    ref = two_launch_block(x, w1, b1, w2, b2)
    diff = np.argwhere(got.view(np.uint16) != ref.view(np.uint16))
    assert diff.size == 0, f"{len(diff)} values differ, first at {diff[0].tolist()}"


def test_resblock_matches_oracle():
    B, H, W, C = 2, 80, 298, 32
    rng = np.random.default_rng(4711)
    x = np.maximum(rng.standard_normal((B, H, W, C), dtype=np.float32), 0).astype(np.float16)
    w1, b1, w2, b2 = _block_params(rng, C)
    announce(f"resblock3x3 vs oracle B={B} H={H} W={W}")
    got = resblock_gpu(x, w1, b1, w2, b2)
    for c in range(B):
        xc = x[c].astype(np.float32).transpose(2, 0, 1)
        t = O.conv2d(xc, w1.astype(np.float32), 1, 1, bias=b1, relu=True).astype(np.float16).astype(np.float32)
        ref = O.conv2d(t, w2.astype(np.float32), 1, 1, bias=b2, residual=xc, relu=True)
        ok, ratio, rel = close_report(got[c].astype(np.float32).transpose(2, 0, 1), ref, CONV_RTOL, CONV_ATOL_RMS)
        assert ok, f"clip {c}: max tol ratio {ratio:.3f}, rel-L2 {rel:.2e}"
        assert rel <= 2e-3, f"clip {c}: rel-L2 {rel:.2e}"


def test_resblock_rejects_bad_arguments():
    L = lib.lib()
    buf = lib.DeviceBuffer(4 * 4 * 64 * 2)
    wb = lib.DeviceBuffer(64 * 9 * 64 * 2)
    bb = lib.DeviceBuffer(64 * 4)
    # 64 channels: no fused kernel
    assert L.vdk_resblock3x3(buf.ptr, 1, 2, 2, 64, wb.ptr, bb.ptr, wb.ptr, bb.ptr, buf.ptr + 4096, None) != 0
    assert "C = 32" in L.vdk_last_error().decode()
    # y overlapping x
    assert L.vdk_resblock3x3(buf.ptr, 1, 4, 4, 32, wb.ptr, bb.ptr, wb.ptr, bb.ptr, buf.ptr + 512, None) != 0
    assert "overlap" in L.vdk_last_error().decode()
    # misaligned output
    assert L.vdk_resblock3x3(buf.ptr, 1, 2, 2, 32, wb.ptr, bb.ptr, wb.ptr, bb.ptr, buf.ptr + 1032, None) != 0
    assert "aligned" in L.vdk_last_error().decode()
