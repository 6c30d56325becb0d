"""moert_attn_decode_noalloc (the attention entry point that allocates nothing, its partials in the library's fixed
device scratch) through the C ABI against moert_attn_decode (the same kernels on buffers it allocates itself): bit for
bit, on two calls in a row, the second with a smaller input (the scratch keeps the first call's contents), and the
refusal of a shape whose partials do not fit the scratch. The test's own device buffers come from the HIP runtime the
library is linked against (libamdhip64.so.7), so that one runtime serves the process."""
import ctypes

import numpy as np
import pytest

import moert

pytestmark = pytest.mark.gpu


class Hip:
    """hipMalloc / hipMemcpy / hipFree / hipDeviceSynchronize of the library's HIP runtime, for the test's buffers."""

    H2D, D2H = 1, 2

    def __init__(self):
        moert.lib()
        self.rt = ctypes.CDLL("libamdhip64.so.7")
        self.rt.hipMalloc.argtypes = [ctypes.POINTER(ctypes.c_void_p), ctypes.c_size_t]
        self.rt.hipMemcpy.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int]
        self.rt.hipFree.argtypes = [ctypes.c_void_p]
        self.bufs = []

    def check(self, rc):
        assert rc == 0, f"HIP error {rc}"

    def upload(self, a: np.ndarray) -> int:
        p = ctypes.c_void_p()
        self.check(self.rt.hipMalloc(ctypes.byref(p), max(a.nbytes, 4)))
        self.bufs.append(p)
        self.check(self.rt.hipMemcpy(p, a.ctypes.data, a.nbytes, self.H2D))
        return p.value

    def download(self, p: int, a: np.ndarray) -> np.ndarray:
        self.check(self.rt.hipMemcpy(a.ctypes.data, ctypes.c_void_p(p), a.nbytes, self.D2H))
        return a

    def sync(self):
        self.check(self.rt.hipDeviceSynchronize())

    def free(self):
        for p in self.bufs:
            self.rt.hipFree(p)
        self.bufs = []


def _case(hip, heads, kv_heads, max_len, length, tps, seed):
    rng = np.random.default_rng(seed)
    q = rng.normal(size=heads * 64).astype(np.float32)
    k = moert.synth_fp16(seed, 1, kv_heads * max_len * 64).reshape(kv_heads, max_len, 64)
    v = moert.synth_fp16(seed, 2, kv_heads * max_len * 64).reshape(kv_heads, max_len, 64)
    scale = 0.125
    want = moert.attn_decode(q, k, v, heads, kv_heads, max_len, length, scale, tps)
    qd, kd, vd = hip.upload(q), hip.upload(k), hip.upload(v)
    od = hip.upload(np.full(heads * 64, np.nan, np.float32))
    moert.attn_decode_noalloc(qd, kd, vd, heads, kv_heads, max_len, length, scale, tps, od, 0)
    hip.sync()
    return hip.download(od, np.empty(heads * 64, np.float32)), want


def test_attention_without_allocation_equals_the_allocating_entry_point(gpu):
    hip = Hip()
    try:
        print("[case] noalloc 3B shape: 24 heads / 8 kv, max_len 4416, len 4100, 3 tiles per split", flush=True)
        got, want = _case(hip, 24, 8, 4416, 4100, 3, 11)
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
        print("[case] noalloc smaller: 4 heads / 2 kv, max_len 256, len 70, 1 tile per split", flush=True)
        got, want = _case(hip, 4, 2, 256, 70, 1, 12)
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    finally:
        hip.free()


def test_attention_without_allocation_refuses_partials_beyond_the_scratch(gpu):
    hip = Hip()
    try:
        p = hip.upload(np.zeros(16, np.float32))
        with pytest.raises(moert.MoertError) as e:  # 128 heads x 64 splits > 64 x 64: refused before any launch
            moert.attn_decode_noalloc(p, p, p, 128, 32, 4096, 100, 0.125, 1, p, 0)
        assert e.value.code == moert.E_CONFIG
    finally:
        hip.free()
