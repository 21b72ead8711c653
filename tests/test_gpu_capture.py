"""A call that would grow one of the context's buffers while its stream is
being captured into a graph fails with CPV_EUNSUPPORTED and records nothing
(a capture may hold no synchronisation, allocation or memset); run outside the
capture, the same call grows the buffer and is bit-exact against the oracle.
The capture goes through the HIP runtime directly (hipStreamBeginCapture)."""
import ctypes

import numpy as np
import pytest
import torch

from oracle import cpvo

pytestmark = pytest.mark.gpu

CAPTURE_RELAXED = 2   # hipStreamCaptureModeRelaxed


def _hip():
    hip = ctypes.CDLL("libamdhip64.so")
    for name, args in (("hipStreamCreate", [ctypes.POINTER(ctypes.c_void_p)]),
                       ("hipStreamBeginCapture", [ctypes.c_void_p, ctypes.c_int]),
                       ("hipStreamEndCapture", [ctypes.c_void_p, ctypes.POINTER(ctypes.c_void_p)]),
                       ("hipGraphDestroy", [ctypes.c_void_p]),
                       ("hipStreamSynchronize", [ctypes.c_void_p]),
                       ("hipStreamDestroy", [ctypes.c_void_p])):
        getattr(hip, name).argtypes = args
        getattr(hip, name).restype = ctypes.c_int
    return hip


def test_buffer_growth_is_refused_inside_a_capture():
    from codpiece_amd import _lib
    from codpiece_amd.runtime import Context
    ctx = Context(0)
    hip = _hip()
    rng = np.random.default_rng(4)
    # a small GEMM sizes the workspace and the accumulator
    q1 = cpvo.quantize(cpvo.Q4_K, rng.normal(0, 0.02, size=(256, 1024)).astype(np.float32))
    w1 = ctx.upload_weight(cpvo.Q4_K, q1, 256, 1024)
    x1 = rng.normal(0, 1, size=(5, 1024)).astype(np.float32)
    ctx.qgemm(w1, torch.from_numpy(x1).cuda())
    torch.cuda.synchronize()
    # a tall one needs the split-K accumulator to grow past its first 16 MiB
    # (16 rows x 151,936 outputs x 8 bytes = 19.4 MB)
    n, k, m = 151936, 256, 16
    q2 = cpvo.quantize(cpvo.Q4_K, rng.normal(0, 0.02, size=(n, k)).astype(np.float32))
    w2 = ctx.upload_weight(cpvo.Q4_K, q2, n, k)
    x2 = torch.from_numpy(rng.normal(0, 1, size=(m, k)).astype(np.float32)).cuda()
    y2 = torch.zeros((m, n), dtype=torch.float32, device="cuda")
    torch.cuda.synchronize()
    stream = ctypes.c_void_p()
    assert hip.hipStreamCreate(ctypes.byref(stream)) == 0
    assert ctx.lib.cpv_set_stream(ctx.h, stream) == _lib.CPV_OK
    assert hip.hipStreamBeginCapture(stream, CAPTURE_RELAXED) == 0
    st = ctx.lib.cpv_qgemm(ctx.h, w2.h, ctypes.c_void_p(x2.data_ptr()), m, ctypes.c_void_p(y2.data_ptr()))
    graph = ctypes.c_void_p()
    end = hip.hipStreamEndCapture(stream, ctypes.byref(graph))
    if graph.value:
        hip.hipGraphDestroy(graph)
    msg = ctx.lib.cpv_last_error(ctx.h).decode()
    assert st == _lib.CPV_EUNSUPPORTED and "captured" in msg, (st, msg)
    assert end == 0
    # outside the capture the call grows the buffers and is exact
    assert ctx.lib.cpv_qgemm(ctx.h, w2.h, ctypes.c_void_p(x2.data_ptr()), m,
                             ctypes.c_void_p(y2.data_ptr())) == _lib.CPV_OK
    assert hip.hipStreamSynchronize(stream) == 0
    ref = cpvo.qgemm(cpvo.Q4_K, q2, x2.cpu().numpy())
    assert np.array_equal(y2.cpu().numpy().view(np.uint32), ref.view(np.uint32))
    ctx.use_stream(torch.cuda.current_stream())
    assert hip.hipStreamDestroy(stream) == 0
    w1.free()
    w2.free()
    ctx.close()
