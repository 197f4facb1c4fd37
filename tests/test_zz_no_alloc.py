"""gs_knn_meandist3_noalloc (the allocation-free distCUDA2, workspace in the
library's per-device scratch array) against gs_knn_meandist3 (caller
workspace), through the C ABI: bit-identical on two calls in a row, the
second on a smaller input (the scratch keeps the first call's contents), and
sizes above the limit are rejected with an error."""
import ctypes as C

import numpy as np
import pytest
import torch

from blitzgs_amd import _lib, synth

pytestmark = pytest.mark.gpu

LIMIT = 1 << 20


def _stream():
    return C.c_void_p(torch.cuda.current_stream().cuda_stream)


def _with_workspace(pts):
    lib = _lib.load()
    P = pts.shape[0]
    out = torch.empty(P, device="cuda")
    ws = torch.empty(lib.gs_knn_workspace_bytes(P), device="cuda", dtype=torch.uint8)
    _lib.check(lib.gs_knn_meandist3(P, _lib.ptr(pts), _lib.ptr(out), _lib.ptr(ws), _stream()), "gs_knn_meandist3")
    return out.cpu().numpy()


def _noalloc(pts):
    lib = _lib.load()
    P = pts.shape[0]
    out = torch.full((P,), float("nan"), device="cuda")
    torch.cuda.synchronize()
    _lib.check(lib.gs_knn_meandist3_noalloc(P, _lib.ptr(pts), _lib.ptr(out), _stream()), "gs_knn_meandist3_noalloc")
    return out.cpu().numpy()


def test_noalloc_knn_matches_workspace_entry_point(gpu):
    big = synth.config4_points(P=LIMIT)                           # the largest allowed size
    rng = np.random.default_rng(8)
    small = rng.uniform(-3.0, 3.0, (70_001, 3)).astype(np.float32)
    small[:50] = small[50:100]                                    # duplicates: distance 0
    for name, pts in (("first call, 2^20 points", big), ("second call, smaller input", small)):
        d = torch.as_tensor(pts, device="cuda")
        got, ref = _noalloc(d), _with_workspace(d)
        assert np.array_equal(got.view(np.uint32), ref.view(np.uint32)), name
        assert np.isfinite(got).all(), name


def test_noalloc_knn_limits(gpu):
    lib = _lib.load()
    x = torch.zeros((4, 3), device="cuda")
    y = torch.empty(4, device="cuda")
    rc = lib.gs_knn_meandist3_noalloc(LIMIT + 1, _lib.ptr(x), _lib.ptr(y), _stream())
    assert rc != 0 and b"allocation-free limit" in lib.gs_last_error()
    assert lib.gs_knn_meandist3_noalloc(0, None, None, _stream()) == 0
    # three points: the missing neighbours keep FLT_MAX, as in the reference
    p3 = torch.as_tensor(np.eye(3, dtype=np.float32), device="cuda")
    assert np.array_equal(_noalloc(p3).view(np.uint32), _with_workspace(p3).view(np.uint32))


def test_noalloc_knn_from_two_host_threads(gpu):
    # two host threads, each on a stream of its own, call the entry point at
    # the same time on different inputs: the per-device lock runs the calls
    # one after another, so every result equals the workspace entry point's
    import threading
    rng = np.random.default_rng(12)
    inputs = [torch.as_tensor(rng.uniform(-2.0, 2.0, (n, 3)).astype(np.float32), device="cuda")
              for n in (300_000, 200_003)]
    refs = [_with_workspace(d) for d in inputs]
    lib = _lib.load()
    results, errors = [[], []], []

    def worker(k):
        try:
            s = torch.cuda.Stream()
            d = inputs[k]
            with torch.cuda.stream(s):
                for _ in range(4):
                    out = torch.full((d.shape[0],), float("nan"), device="cuda")
                    rc = lib.gs_knn_meandist3_noalloc(d.shape[0], _lib.ptr(d), _lib.ptr(out),
                                                      C.c_void_p(s.cuda_stream))
                    if rc != 0:
                        errors.append(lib.gs_last_error())
                        return
                    results[k].append(out.cpu().numpy())
        except Exception as e:   # reported below
            errors.append(repr(e))

    torch.cuda.synchronize()
    threads = [threading.Thread(target=worker, args=(k,)) for k in (0, 1)]
    for t in threads:
        t.start()
    for t in threads:
        t.join(timeout=120)
    assert not errors, errors
    for k in (0, 1):
        assert len(results[k]) == 4
        for got in results[k]:
            assert np.array_equal(got.view(np.uint32), refs[k].view(np.uint32)), k
