"""vdk_linear_ex_noalloc: the FC entry point that allocates nothing (its split-K
partials live in a fixed per-GPU scratch array) must give, bit for bit, what
vdk_linear_ex gives with a caller workspace, on two calls in a row (the second
smaller, over the scratch the first left behind), and refuse shapes whose
partials exceed the array before launching anything."""
import numpy as np
import pytest

from gpu_util import announce, device_ok
from vdamd import lib

pytestmark = pytest.mark.gpu

SCRATCH_BYTES = 4 << 20   # VDK_LINEAR_SCRATCH_BYTES in include/vdk.h


def _case(B, I, E, seed):
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((B, I)).astype(np.float32)
    w = (rng.standard_normal((E, I)) / np.sqrt(I)).astype(np.float32)
    b = (0.1 * rng.standard_normal(E)).astype(np.float32)
    mv = (0.05 * rng.standard_normal(E)).astype(np.float32)
    return x, w, b, mv


def _run_pair(L, B, I, E, act, seed):
    x, w, b, mv = _case(B, I, E, seed)
    dx, dw, db, dm = (lib.DeviceBuffer.from_array(a) for a in (x, w, b, mv))
    y_ws, y_na = lib.DeviceBuffer(B * E * 4), lib.DeviceBuffer(B * E * 4)
    wsz = L.vdk_linear_workspace_size(B, I, E)
    assert 0 < wsz <= SCRATCH_BYTES
    work = lib.DeviceBuffer(wsz)
    announce(f"linear_noalloc B={B} in={I} out={E} act={act} (workspace {wsz} B)")
    lib.check(L.vdk_linear_ex(dx.ptr, B, I, dw.ptr, db.ptr, dm.ptr, E, act, y_ws.ptr, work.ptr, wsz, None))
    lib.check(L.vdk_linear_ex_noalloc(dx.ptr, B, I, dw.ptr, db.ptr, dm.ptr, E, act, y_na.ptr, None))
    lib.check(L.vdk_synchronize())
    got, want = y_na.to_array(np.float32, (B, E)), y_ws.to_array(np.float32, (B, E))
    assert np.array_equal(got, want)
    ref = x.astype(np.float64) @ w.astype(np.float64).T + b - mv
    ref = {0: ref, 1: np.maximum(ref, 0), 5: np.tanh(ref)}[act]
    np.testing.assert_allclose(got, ref, rtol=2e-5, atol=2e-5)


@pytest.mark.skipif(not device_ok(), reason="no HIP device")
def test_noalloc_linear_matches_workspace_linear_twice():
    L = lib.lib()
    # the ResNet34 embedding FC of a 64-clip batch (5120 -> 256, 40 slices),
    # then a smaller ragged product over what the first call left behind
    _run_pair(L, 64, 5120, 256, 0, 1)
    _run_pair(L, 3, 769, 64, 1, 2)
    _run_pair(L, 64, 5120, 256, 5, 3)


@pytest.mark.skipif(not device_ok(), reason="no HIP device")
def test_noalloc_linear_rejects_oversized_partials():
    L = lib.lib()
    B, I, E = 1024, 5120, 256            # 40 slices x 1024 x 256 floats = 40 MiB
    assert L.vdk_linear_workspace_size(B, I, E) > SCRATCH_BYTES
    # operands at their full sizes (20 + 5 + 1 MiB), so that a regressed size
    # guard computes a product over valid memory and fails the assertion
    dx, dw, dy = lib.DeviceBuffer(4 * B * I), lib.DeviceBuffer(4 * I * E), lib.DeviceBuffer(4 * B * E)
    rc = L.vdk_linear_ex_noalloc(dx.ptr, B, I, dw.ptr, None, None, E, 0, dy.ptr, None)
    err = L.vdk_last_error()
    lib.check(L.vdk_synchronize())
    assert rc != 0
    assert b"scratch" in err
