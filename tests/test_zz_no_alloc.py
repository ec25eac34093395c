"""The allocation-free entry point mh_resize_noalloc, through the C ABI, against mh_resize (the entry point it
varies) and the CPU oracle's INTER_AREA: bit for bit, on two calls in a row, the second with fewer images; its
first call in a fresh process made under HIP graph capture, followed by an uncaptured call and several replays;
and its refusals (n out of range, null buffers)."""
import ctypes
import os
import subprocess
import sys

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


# Run in a fresh process, so that the captured call is the process's first call of the entry point.
_CAPTURE = r"""
import ctypes, sys
import numpy as np
import torch
sys.path.insert(0, sys.argv[1])
from fast_mario_env_amd import _native
L = ctypes.CDLL(_native.lib_path())
L.mh_last_error.restype = ctypes.c_char_p
for f in (L.mh_resize, L.mh_resize_noalloc):
    f.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int, ctypes.c_void_p]
n = 11
rng = np.random.default_rng(5)
src = torch.from_numpy(rng.integers(0, 256, (n, 240, 256), np.uint8)).cuda()
out = torch.zeros(n, 84, 84, dtype=torch.uint8, device="cuda")
torch.cuda.synchronize()
g = torch.cuda.CUDAGraph()
with torch.cuda.graph(g):
    rc = L.mh_resize_noalloc(src.data_ptr(), out.data_ptr(), n, torch.cuda.current_stream().cuda_stream)
assert rc == 0, L.mh_last_error()
stream = torch.cuda.current_stream().cuda_stream
# an uncaptured call before the graph has ever run, against mh_resize
a = torch.zeros_like(out)
want = torch.zeros_like(out)
assert L.mh_resize_noalloc(src.data_ptr(), a.data_ptr(), n, stream) == 0, L.mh_last_error()
assert L.mh_resize(src.data_ptr(), want.data_ptr(), n, stream) == 0, L.mh_last_error()
torch.cuda.synchronize()
assert torch.equal(a, want), "uncaptured call after a captured first call"
assert not torch.equal(want, torch.zeros_like(want))
# replays, with new images and eager work between them, each against an eager mh_resize
for rep in range(3):
    src.copy_(torch.from_numpy(rng.integers(0, 256, (n, 240, 256), np.uint8)).cuda())
    assert L.mh_resize(src.data_ptr(), want.data_ptr(), n, stream) == 0, L.mh_last_error()
    out.zero_()
    torch.cuda.synchronize()
    g.replay()
    torch.cuda.synchronize()
    assert torch.equal(out, want), ("replay", rep)
print("capture ok")
"""


def test_resize_noalloc_first_call_under_capture():
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    print("fresh process: first mh_resize_noalloc call under graph capture", flush=True)
    r = subprocess.run([sys.executable, "-c", _CAPTURE, os.path.join(root, "fast-mario-env_amd")],
                       capture_output=True, text=True, timeout=240)
    assert r.returncode == 0 and "capture ok" in r.stdout, (r.returncode, r.stdout[-2000:], r.stderr[-3000:])
