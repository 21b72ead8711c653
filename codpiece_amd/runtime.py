"""Host wrapper over the C ABI: a device context, weight handles, kernel calls.

Device memory is torch tensors on cuda:N (PyTorch-ROCm is only the allocator and
the stream here); every computation runs in libcpv.so.  The context enqueues on
torch's current stream so library calls and torch ops stay ordered.
"""
import ctypes

import numpy as np
import torch

from . import _lib
from ._lib import CpvError, SamplerParams


def _ptr(t):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


class Context:
    """One device, one stream (cpv_init / cpv_set_stream)."""

    def __init__(self, device=0):
        if not torch.cuda.is_available():
            raise RuntimeError("codpiece_amd needs a ROCm GPU (torch.cuda.is_available() is False)")
        self.lib = _lib.load()
        self.device = device
        self.torch_device = torch.device("cuda", device)
        h = ctypes.c_void_p()
        st = self.lib.cpv_init(device, ctypes.byref(h))
        if st != _lib.CPV_OK:
            raise CpvError(st, f"cpv_init({device}) failed")
        self.h = h
        self.use_stream(torch.cuda.current_stream(self.torch_device))

    def use_stream(self, stream):
        self._check(self.lib.cpv_set_stream(self.h, ctypes.c_void_p(stream.cuda_stream)))
        self.stream = stream

    def _check(self, st):
        if st != _lib.CPV_OK:
            raise CpvError(st, self.lib.cpv_last_error(self.h).decode())

    def sync(self):
        self._check(self.lib.cpv_sync(self.h))

    def profile_start(self):
        """Time every GEMM / attention launch with HIP events until profile_stop."""
        self._check(self.lib.cpv_profile_start(self.h))

    def profile_stop(self):
        """{class name: (launches, ms, algorithmic bytes)} since profile_start."""
        out = (_lib.ProfStat * _lib.PROF_CLASSES)()
        self._check(self.lib.cpv_profile_stop(self.h, out))
        return {name: (out[i].launches, out[i].ms, out[i].bytes) for i, name in enumerate(_lib.PROF_NAMES)}

    def profile_replay(self, cls_name, reps=5):
        """(ms per launch, algorithmic bytes per launch) of the class's recorded
        launches replayed back to back."""
        ms, b = ctypes.c_double(), ctypes.c_double()
        self._check(self.lib.cpv_profile_replay(self.h, _lib.PROF_NAMES.index(cls_name), reps, ctypes.byref(ms),
                                                ctypes.byref(b)))
        return ms.value, b.value

    def close(self):
        if getattr(self, "h", None):
            self.lib.cpv_free(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    # ---- weights
    def upload_weight(self, qtype, data, n_rows, k):
        """data: ggml block bytes of n_rows rows (numpy uint8) or a cuda uint8 tensor."""
        out = ctypes.c_void_p()
        if isinstance(data, torch.Tensor):
            assert data.is_cuda and data.dtype == torch.uint8
            st = self.lib.cpv_weight_from_device(self.h, qtype, _ptr(data), n_rows, k, ctypes.byref(out))
        else:
            arr = np.ascontiguousarray(data, dtype=np.uint8)
            st = self.lib.cpv_weight_upload(self.h, qtype, arr.ctypes.data_as(ctypes.c_void_p), n_rows, k,
                                            ctypes.byref(out))
        self._check(st)
        return Weight(self, out, qtype, n_rows, k)

    # ---- kernels
    def qgemm(self, w, x, y=None):
        """y[m][n] = x[m] . dequant(w[n]) (ggml_mul_mat(w, x))."""
        assert x.is_cuda and x.dtype == torch.float32 and x.is_contiguous() and x.shape[1] == w.k
        if y is None:
            y = torch.empty((x.shape[0], w.n), dtype=torch.float32, device=x.device)
        self._check(self.lib.cpv_qgemm(self.h, w.h, _ptr(x), x.shape[0], _ptr(y)))
        return y

    def qgemm_noalloc(self, w, x, y):
        """qgemm into a caller-allocated y through the allocation-free entry
        point (per-device scratch; m <= 16)."""
        assert x.is_cuda and x.dtype == torch.float32 and x.is_contiguous() and x.shape[1] == w.k
        assert y.is_cuda and y.dtype == torch.float32 and y.is_contiguous() and y.shape == (x.shape[0], w.n)
        self._check(self.lib.cpv_qgemm_noalloc(self.h, w.h, _ptr(x), x.shape[0], _ptr(y)))
        return y

    def get_rows(self, w, rows, out=None):
        rows = rows.to(torch.int32).contiguous()
        if out is None:
            out = torch.empty((rows.numel(), w.k), dtype=torch.float32, device=rows.device)
        self._check(self.lib.cpv_get_rows(self.h, w.h, _ptr(rows), rows.numel(), _ptr(out)))
        return out

    def argmax_rows(self, x, noise=None, out=None):
        x = x.contiguous()
        rows, n = x.shape
        if out is None:
            out = torch.empty(rows, dtype=torch.int32, device=x.device)
        self._check(self.lib.cpv_argmax_rows(self.h, _ptr(x), _ptr(noise), rows, n, _ptr(out)))
        return out

    def redraft_gate(self, logits, p_min):
        """cpv_redraft_gate over logits [rows][v]: (argmax [rows], keep [rows])
        int32 device tensors; keep = 0 where the softmax peak 1 / lse is below
        p_min (lse the index-order f32 sum, engine.rs:2598-2606)."""
        logits = logits.contiguous()
        rows, v = logits.shape
        am = torch.empty(rows, dtype=torch.int32, device=logits.device)
        keep = torch.empty(rows, dtype=torch.int32, device=logits.device)
        self._check(self.lib.cpv_redraft_gate(self.h, _ptr(logits), rows, v, float(p_min), _ptr(am), _ptr(keep)))
        return am, keep

    def attn(self, q, k_cache, v_cache_t, n_past, parent, h_kv, scale, out=None):
        """q [t][h][d] f32; k_cache [n_ctx][h_kv*d] and v_cache_t [h_kv*d][v_stride], 16-bit tensors."""
        t, h, d = q.shape
        if out is None:
            out = torch.empty((t, h * d), dtype=torch.float32, device=q.device)
        par = None if parent is None else parent.to(torch.int32).contiguous()
        self._check(self.lib.cpv_attn(self.h, _ptr(q.contiguous()), _ptr(k_cache), _ptr(v_cache_t),
                                      v_cache_t.shape[1], n_past, _ptr(par), t, h, h_kv, d, scale, _ptr(out)))
        return out

    def distribution(self, logits, params, hist=None):
        """Sampler::distribution of each row of logits [rows][v]: (ids, probs, n) device tensors."""
        logits = logits.contiguous()
        rows, v = logits.shape
        ids = torch.empty((rows, v), dtype=torch.int32, device=logits.device)
        probs = torch.empty((rows, v), dtype=torch.float32, device=logits.device)
        n = torch.empty(rows, dtype=torch.int32, device=logits.device)
        h = None if hist is None else hist.to(torch.int32).contiguous()
        self._check(self.lib.cpv_distribution(self.h, _ptr(logits), rows, v, ctypes.byref(params), _ptr(h),
                                              0 if h is None else h.shape[1], _ptr(ids), _ptr(probs), _ptr(n)))
        return ids, probs, n

    def spec_accept(self, p_logits, draft, params, mode, u=None, q_logits=None, noise=None, hist=None,
                    philox_seed=0, philox_round=0, out_tok=None, out_n=None):
        b, k1, v = p_logits.shape
        k = k1 - 1
        if out_tok is None:
            out_tok = torch.full((b, k1), -1, dtype=torch.int32, device=p_logits.device)
        if out_n is None:
            out_n = torch.empty(b, dtype=torch.int32, device=p_logits.device)
        hl = 0 if hist is None else hist.shape[1]
        self._check(self.lib.cpv_spec_accept(
            self.h, _ptr(p_logits), _ptr(q_logits), _ptr(draft.to(torch.int32).contiguous()), b, k, v,
            ctypes.byref(params), mode, _ptr(u), philox_seed, philox_round, _ptr(noise),
            _ptr(None if hist is None else hist.to(torch.int32).contiguous()), hl, _ptr(out_tok), _ptr(out_n)))
        return out_tok, out_n


class Weight:
    def __init__(self, ctx, h, qtype, n, k):
        self.ctx, self.h, self.qtype, self.n, self.k = ctx, h, qtype, n, k

    def info(self):
        t, n, k, b = ctypes.c_int(), ctypes.c_int64(), ctypes.c_int64(), ctypes.c_int64()
        self.ctx._check(self.ctx.lib.cpv_weight_info(self.h, ctypes.byref(t), ctypes.byref(n), ctypes.byref(k),
                                                     ctypes.byref(b)))
        return t.value, n.value, k.value, b.value

    def free(self):
        if self.h:
            self.ctx.lib.cpv_weight_free(self.h)
            self.h = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


__all__ = ["Context", "Weight", "SamplerParams", "CpvError"]
