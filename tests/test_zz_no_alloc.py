"""pdefa_amd_ops_matmul_noalloc (device buffers in a static scratch array,
no allocation) through the C ABI against engine_ops_matmul, whose kernels
and launch shapes it shares: the same bits, on consecutive calls of
decreasing size (the second finds the first one's data in the array)."""
import ctypes as C

import numpy as np
import pytest

from pdefa_amd import native

pytestmark = pytest.mark.gpu


def _pair(a_shape, b_shape, seed):
    rng = np.random.default_rng(seed)
    a = rng.standard_normal(a_shape, dtype=np.float32)
    b = rng.standard_normal(b_shape, dtype=np.float32)
    out = np.zeros(a_shape[:-1] + (b_shape[-1],), np.float32)
    return a, b, out


def _check(a, b, out, what):
    got = native.matmul_into(a, b, out, noalloc=True)
    want = native.matmul_into(a, b, out)
    assert np.array_equal(got, want), f"{what}: differs from engine_ops_matmul"
    ref = np.matmul(a.astype(np.float64), b.astype(np.float64))
    err = np.abs(got - ref)
    assert err.max() <= 1e-3, f"{what}: max abs err {err.max():.3e} against float64"
    print(f"{what}: equal to engine_ops_matmul, max abs err {err.max():.3e} against float64", flush=True)


def test_noalloc_matmul_matches_ops_matmul_on_two_calls():
    print("[case] ops_matmul_noalloc 512x512x512 then 100x37x70", flush=True)
    _check(*_pair((512, 512), (512, 512), 42), "512^3")
    _check(*_pair((100, 37), (37, 70), 7), "100x37 @ 37x70 (second, smaller call)")


def test_noalloc_matmul_batched_and_split_k():
    """Batched product (one GEMM per batch, the array reused by each) and a
    deep-K shape whose launch splits K across workgroups (partials in the
    array)."""
    print("[case] ops_matmul_noalloc batched 3x64x96 @ 96x40, then 16x4096 @ 4096x16", flush=True)
    _check(*_pair((3, 64, 96), (96, 40), 3), "batched, shared B")
    _check(*_pair((16, 4096), (4096, 16), 5), "deep K")


def test_noalloc_matmul_rejects_oversize_and_keeps_ops_rules():
    print("[case] ops_matmul_noalloc 2048^3 (over the scratch) and a shape mismatch", flush=True)
    a, b, out = _pair((2048, 2048), (2048, 2048), 1)
    with pytest.raises(native.NativeError) as e:
        native.matmul_into(a, b, out, noalloc=True)
    assert e.value.status == native.ENGINE_ERR_INVALID_ARG and "static scratch array" in str(e.value)
    a, b, _ = _pair((4, 5), (6, 3), 2)
    sentinel = np.full((4, 3), -7.25, np.float32)
    np.testing.assert_array_equal(native.matmul_into(a, b, sentinel, noalloc=True), sentinel)
    # the array still serves the next call
    _check(*_pair((33, 65), (65, 17), 9), "after the rejected call")


def _device_free_bytes():
    """hipMemGetInfo's free bytes of the current device (the HIP runtime the
    library is linked against)."""
    native.lib()
    hip = C.CDLL("libamdhip64.so")
    free, total = C.c_size_t(), C.c_size_t()
    assert hip.hipMemGetInfo(C.byref(free), C.byref(total)) == 0
    return free.value


def test_noalloc_matmul_allocates_no_device_memory():
    """A call of a shape larger than any earlier one leaves the device's free
    memory unchanged; engine_ops_matmul on the same shape grows its scratch."""
    print("[case] ops_matmul_noalloc 1200x1024 @ 1024x1100: device free memory", flush=True)
    _check(*_pair((64, 64), (64, 64), 11), "warm-up")
    a, b, out = _pair((1200, 1024), (1024, 1100), 12)
    before = _device_free_bytes()
    got = native.matmul_into(a, b, out, noalloc=True)
    after = _device_free_bytes()
    assert after == before, f"the no-allocation call changed free device memory by {before - after} bytes"
    want = native.matmul_into(a, b, out)
    grown = _device_free_bytes()
    assert grown < after, "engine_ops_matmul allocated nothing for the larger shape"
    assert np.array_equal(got, want)
    print(f"free device memory unchanged by the no-allocation call; engine_ops_matmul took "
          f"{(after - grown) / 2**20:.1f} MiB", flush=True)
