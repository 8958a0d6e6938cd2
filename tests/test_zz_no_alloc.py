"""The attention entry point that allocates nothing (yhip_attention_noalloc) against the one that
allocates (yhip_test_attention): same kernels, so the outputs must be bit-identical, over two calls
in a row on one GPU (the second smaller, so stale scratch contents would show), in sink mode (the K
cache is rewritten in place) and on both attention kernels. The test's device buffers come from the
HIP runtime the library itself links (libamdhip64.so.7), through ctypes."""
import ctypes

import numpy as np
import pytest

from oracle import binding as O
from tests.util import f16

pytestmark = pytest.mark.gpu


def hip():
    from yalm_amd import hip as H
    H.lib()
    return H


class DeviceBuffers:
    """hipMalloc'd copies of host arrays (test side only), freed on exit."""

    def __init__(self):
        hip()  # the library is loaded first, so this resolves to the runtime it uses
        self.rt = ctypes.CDLL("libamdhip64.so.7")
        self.rt.hipMalloc.argtypes = [ctypes.POINTER(ctypes.c_void_p), ctypes.c_size_t]
        self.rt.hipMemcpy.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int]
        self.rt.hipFree.argtypes = [ctypes.c_void_p]
        self.ptrs = []

    def put(self, a):
        a = np.ascontiguousarray(a)
        p = ctypes.c_void_p()
        assert self.rt.hipMalloc(ctypes.byref(p), max(a.nbytes, 4)) == 0
        self.ptrs.append(p)
        assert self.rt.hipMemcpy(p, a.ctypes.data_as(ctypes.c_void_p), a.nbytes, 1) == 0  # host to device
        return p

    def get(self, p, like):
        out = np.empty_like(like)
        assert self.rt.hipDeviceSynchronize() == 0
        assert self.rt.hipMemcpy(out.ctypes.data_as(ctypes.c_void_p), p, out.nbytes, 2) == 0  # device to host
        return out

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.rt.hipDeviceSynchronize()
        for p in self.ptrs:
            self.rt.hipFree(p)


def _noalloc(q, kb, vb, hd, pos, msl, nh, nkv, nsplit):
    H = hip()
    with DeviceBuffers() as d:
        dq, dk, dv = d.put(np.asarray(q, np.float32)), d.put(np.asarray(kb, np.uint16)), d.put(np.asarray(vb, np.uint16))
        nan = np.full(nh * hd, np.nan, np.float32)
        dout = d.put(nan)
        rc = H.lib().yhip_attention_noalloc(dq, dk, dv, hd, pos, msl, nh, nkv, nsplit, ctypes.c_float(1e6), hd,
                                            dout, None)
        if rc != 0:
            raise H.HipError(H.lib().yhip_last_error(None).decode())
        return d.get(dout, nan), d.get(dk, np.asarray(kb, np.uint16))


# (hd, nh, nkv, msl, pos, nsplit): a long Mistral-shape call, then smaller ones; the last two are
# in sink mode (pos >= max_seq_len)
CALLS = [(128, 32, 8, 4096, 3200, 0), (32, 8, 2, 512, 299, 5), (128, 32, 8, 1024, 1030, 0), (32, 8, 2, 64, 70, 3)]


@pytest.mark.parametrize("mfma", [1, 0], ids=["mfma", "simt"])
def test_noalloc_attention_matches_the_allocating_entry_point(mfma):
    H = hip()
    H.set_attn_mfma(mfma)
    try:
        for i, (hd, nh, nkv, msl, pos, nsplit) in enumerate(CALLS):
            rng = np.random.default_rng(100 + i)
            kb = f16(rng.standard_normal(nkv * hd * msl))
            vb = f16(rng.standard_normal(nkv * hd * msl))
            q = rng.standard_normal(nh * hd).astype(np.float32)
            want, k_want = H.attention(q, kb, vb, hd, pos, msl, nh, nkv, nsplit=nsplit)
            got, k_got = _noalloc(q, kb, vb, hd, pos, msl, nh, nkv, nsplit)
            assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), (i, mfma)
            assert np.array_equal(k_got, k_want), (i, mfma)
            ref, _ = O.mha(q, k_want, vb, hd, min(pos + 1, msl), msl, nh, nkv)
            assert np.linalg.norm(got - ref) <= 1e-5 * np.linalg.norm(ref)
    finally:
        H.set_attn_mfma(1)


def test_noalloc_attention_rejects_sizes_beyond_its_scratch():
    H = hip()
    # 64 query heads x 64 slices x 130 floats = 2.1 MB of partials > 1 MiB: refused on the host,
    # before anything is launched
    hd, nh, nkv, msl = 128, 64, 8, 4096
    with DeviceBuffers() as d:
        dq = d.put(np.zeros(nh * hd, np.float32))
        dk = d.put(np.zeros(nkv * hd * msl, np.uint16))
        dout = d.put(np.zeros(nh * hd, np.float32))
        rc = H.lib().yhip_attention_noalloc(dq, dk, dk, hd, 100, msl, nh, nkv, 64, ctypes.c_float(1e6), hd, dout, None)
        assert rc == -1
        assert b"1 MiB" in H.lib().yhip_last_error(None)
