"""Device-memory plumbing for GPU tests (torch is only the allocator/stream)."""
import ctypes

import numpy as np


def to_dev(a: np.ndarray):
    import torch
    t = torch.from_numpy(np.ascontiguousarray(a)).to("cuda:0")
    return t


def empty(n, dtype):
    import torch
    return torch.empty(n, dtype=dtype, device="cuda:0")


def ptr(t):
    return ctypes.c_void_p(t.data_ptr())


def stream():
    import torch
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


def call(fn, *args):
    import torch
    print(f"[gpu] {fn.__name__} args={[a for a in args if isinstance(a, int)]}", flush=True)
    rc = fn(*args, stream())
    assert rc == 0, f"{fn.__name__} returned hipError {rc}"
    torch.cuda.synchronize()


def host(t):
    return t.cpu().numpy()


def gemv_error(y, ref):
    """(max |y-ref| / max|ref|, max elementwise |y-ref| / (1e-6*max|ref| + 1e-5*|ref|))."""
    y = y.astype(np.float64)
    scale = np.abs(ref).max()
    diff = np.abs(y - ref)
    return diff.max() / scale, (diff / (1e-6 * scale + 1e-5 * np.abs(ref))).max()
