"""The allocation-free entry point mh_resize_noalloc, through the C ABI, against mh_resize (the entry point it
varies) and the CPU oracle's INTER_AREA: bit for bit, on two calls in a row, the second with fewer images, plus
its refusals (n out of range, null buffers)."""
import ctypes

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def _lib():
    from fast_mario_env_amd import _native
    L = ctypes.CDLL(_native.lib_path())
    L.mh_last_error.restype = ctypes.c_char_p
    for f in (L.mh_resize, L.mh_resize_noalloc):
        f.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int, ctypes.c_void_p]
    return L


def _images(rng, n):
    imgs = rng.integers(0, 256, (n, 240, 256), np.uint8)
    imgs[::3] = np.repeat(np.repeat(rng.integers(0, 256, (len(imgs[::3]), 30, 32), np.uint8), 8, 1), 8, 2)
    return imgs


def test_resize_noalloc_matches_resize_and_oracle():
    import torch

    from cpu_libs import oracle
    L = _lib()
    stream = torch.cuda.current_stream().cuda_stream
    rng = np.random.default_rng(21)
    for n in (37, 5):                                   # the second call smaller than the first
        src = torch.from_numpy(_images(rng, n)).cuda()
        a = torch.full((n, 84, 84), 7, dtype=torch.uint8, device="cuda")
        b = torch.full((n, 84, 84), 9, dtype=torch.uint8, device="cuda")
        assert L.mh_resize_noalloc(src.data_ptr(), a.data_ptr(), n, stream) == 0, L.mh_last_error()
        assert L.mh_resize(src.data_ptr(), b.data_ptr(), n, stream) == 0, L.mh_last_error()
        torch.cuda.synchronize()
        assert torch.equal(a, b), n
        host = src.cpu().numpy()
        out = a.cpu().numpy()
        for i in range(0, n, 4):
            want = np.zeros((84, 84), np.uint8)
            oracle().or_resize(np.ascontiguousarray(host[i]).ctypes.data, want.ctypes.data)
            assert np.array_equal(out[i], want), (n, i)


def test_resize_noalloc_refusals():
    import torch
    L = _lib()
    src = torch.zeros(1, 240, 256, dtype=torch.uint8, device="cuda")
    dst = torch.zeros(1, 84, 84, dtype=torch.uint8, device="cuda")
    stream = torch.cuda.current_stream().cuda_stream
    for n in (0, -3, 65536):
        assert L.mh_resize_noalloc(src.data_ptr(), dst.data_ptr(), n, stream) == -1
        assert b"1 .. 65535" in L.mh_last_error()
    assert L.mh_resize_noalloc(None, dst.data_ptr(), 1, stream) == -1
    assert b"null" in L.mh_last_error()
    assert L.mh_resize_noalloc(src.data_ptr(), dst.data_ptr(), 1, stream) == 0
    torch.cuda.synchronize()
