"""ctypes view of the CPU oracle (oracle/libcpvo.so).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and
bench.py's cpu_baseline leg as the checker.  The product package never imports
this module.
"""
import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "libcpvo.so")

F32, F16, Q8_0, Q4_K, Q6_K, Q8_K = 0, 1, 8, 12, 14, 15
BLOCK = {F32: 1, F16: 1, Q8_0: 32, Q4_K: 256, Q6_K: 256, Q8_K: 256}
SIZE = {F32: 4, F16: 2, Q8_0: 34, Q4_K: 144, Q6_K: 210, Q8_K: 292}
ACCEPT_GREEDY, ACCEPT_REJECT, ACCEPT_GUMBEL = 0, 1, 2


def build(force=False):
    """Compile the oracle with its own Makefile (gcc, -ffp-contract=off)."""
    if force or not os.path.exists(_LIB_PATH):
        subprocess.run(["make", "-s", "-C", _HERE, "-B" if force else "all"], check=True)
    return _LIB_PATH


class SamplerParams(ctypes.Structure):
    """Mirror of SamplerParams (crates/codpiece-sample/src/lib.rs:29-64)."""
    _fields_ = [
        ("temp", ctypes.c_float),
        ("top_k", ctypes.c_int32),
        ("top_p", ctypes.c_float),
        ("min_p", ctypes.c_float),
        ("min_keep", ctypes.c_int32),
        ("penalty_repeat", ctypes.c_float),
        ("penalty_freq", ctypes.c_float),
        ("penalty_present", ctypes.c_float),
        ("penalty_last_n", ctypes.c_int32),
    ]

    def __init__(self, temp=0.0, top_k=0, top_p=1.0, min_p=0.0, min_keep=1,
                 penalty_repeat=1.0, penalty_freq=0.0, penalty_present=0.0,
                 penalty_last_n=64):
        super().__init__(temp, top_k, top_p, min_p, min_keep, penalty_repeat,
                         penalty_freq, penalty_present, penalty_last_n)


_lib = None


def lib():
    global _lib
    if _lib is None:
        build()
        L = ctypes.CDLL(_LIB_PATH)
        P = ctypes.c_void_p
        i64, i32, f32 = ctypes.c_int64, ctypes.c_int32, ctypes.c_float
        sig = {
            "cpvo_fp32_to_fp16_n": (None, [P, i64, P]),
            "cpvo_fp16_to_fp32_n": (None, [P, i64, P]),
            "cpvo_expf_n": (None, [P, i64, P]),
            "cpvo_expf_vs_libm": (i64, [f32, f32, i64]),
            "cpvo_exp_table": (None, [P]),
            "cpvo_philox4x64": (None, [P, P, P]),
            "cpvo_philox_uniforms": (None, [ctypes.c_uint64, ctypes.c_uint64, ctypes.c_int, ctypes.c_int, P]),
            "cpvo_rng_seed": (None, [ctypes.c_uint64, P]),
            "cpvo_rng_next_u64": (ctypes.c_uint64, [P]),
            "cpvo_rng_next_f32": (f32, [P]),
            "cpvo_quantize": (ctypes.c_int, [ctypes.c_int, P, i64, P]),
            "cpvo_dequantize": (ctypes.c_int, [ctypes.c_int, P, i64, P]),
            "cpvo_quantize_q8_0": (None, [P, i64, P]),
            "cpvo_quantize_q8_K": (None, [P, i64, P]),
            "cpvo_qgemm": (ctypes.c_int, [ctypes.c_int, P, i64, i64, P, i64, P, ctypes.c_int]),
            "cpvo_qgemm_f64": (ctypes.c_int, [ctypes.c_int, P, i64, i64, P, i64, P, ctypes.c_int]),
            "cpvo_qgemm_window": (ctypes.c_int, [ctypes.c_int, i64]),
            "cpvo_mul_mat_f32": (None, [P, i64, i64, P, i64, P]),
            "cpvo_rms_norm": (None, [P, i64, f32, P, P]),
            "cpvo_rope_table": (None, [ctypes.c_int, ctypes.c_int, f32, P]),
            "cpvo_rope_table_sections": (None, [ctypes.c_int, ctypes.c_int, f32, P, P]),
            "cpvo_rope_neox": (None, [P, ctypes.c_int, P]),
            "cpvo_attn": (None, [P, P, P, i64, P, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                 ctypes.c_int, f32, P]),
            "cpvo_attn_f64": (None, [P, P, P, i64, P, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                 ctypes.c_int, f32, P]),
            "cpvo_distribution": (ctypes.c_int, [P, P, ctypes.c_int, P, ctypes.c_int, P, P, P]),
            "cpvo_dist_draw": (i32, [P, P, ctypes.c_int, f32]),
            "cpvo_dist_draw_excluding": (i32, [P, P, ctypes.c_int, i32, f32]),
            "cpvo_dist_prob_of": (f32, [P, P, ctypes.c_int, i32]),
            "cpvo_dist_peak": (f32, [P, ctypes.c_int]),
            "cpvo_sample_coupled": (i32, [P, P, ctypes.c_int, P, ctypes.c_int, P]),
            "cpvo_argmax": (i32, [P, i64]),
            "cpvo_softmax_peak_seq": (f32, [P, i64]),
            "cpvo_spec_accept": (ctypes.c_int, [P, P, P, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                                P, ctypes.c_int, P, P, P, ctypes.c_int, P, P]),
            "cpvo_spec_accept_rng": (ctypes.c_int, [P, P, ctypes.c_int, ctypes.c_int, P, P, P,
                                                    ctypes.c_int, P, P]),
            "cpvo_model_create": (P, [P]),
            "cpvo_model_free": (None, [P]),
            "cpvo_model_set": (ctypes.c_int, [P, ctypes.c_char_p, ctypes.c_int, P, i64, i64]),
            "cpvo_session_create": (P, [P, i64]),
            "cpvo_session_free": (None, [P]),
            "cpvo_session_set_pos": (None, [P, i64, i64]),
            "cpvo_session_get_pos": (None, [P, P, P]),
            "cpvo_session_set_attn_inject": (None, [P, P, i64]),
            "cpvo_session_inject_ratio": (ctypes.c_double, [P]),
            "cpvo_set_fault": (None, [ctypes.c_int]),
            "cpvo_set_attn_f64": (None, [ctypes.c_int]),
            "cpvo_set_smooth": (None, [ctypes.c_int]),
            "cpvo_set_threads": (None, [ctypes.c_int]),
            "cpvo_prefill": (ctypes.c_int, [P, P, ctypes.c_int]),
            "cpvo_verify_step": (ctypes.c_int, [P, P, ctypes.c_int, ctypes.c_int, P, P, P, P, P, P]),
            "cpvo_verify_step_cands": (ctypes.c_int, [P, P, ctypes.c_int, ctypes.c_int, P, P, ctypes.c_int, P, P, P,
                                                      P, P]),
            "cpvo_mtp_draft": (ctypes.c_int, [P, P, i32, i64, P, P]),
            "cpvo_fused_generate": (ctypes.c_int, [P, P, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                                   ctypes.c_int, ctypes.c_int, P, P]),
        }
        for name, (res, args) in sig.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def _p(a):
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


def f32_to_f16_bits(x):
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.shape, dtype=np.uint16)
    lib().cpvo_fp32_to_fp16_n(_p(x), x.size, _p(out))
    return out


def f16_bits_to_f32(h):
    h = np.ascontiguousarray(h, dtype=np.uint16)
    out = np.empty(h.shape, dtype=np.float32)
    lib().cpvo_fp16_to_fp32_n(_p(h), h.size, _p(out))
    return out


def expf(x):
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty_like(x)
    lib().cpvo_expf_n(_p(x), x.size, _p(out))
    return out


def exp_table():
    out = np.empty(32, dtype=np.uint64)
    lib().cpvo_exp_table(_p(out))
    return out


def expf_vs_libm(lo, hi, stride=1):
    return lib().cpvo_expf_vs_libm(lo, hi, stride)


def philox4x64(ctr, key):
    c = np.ascontiguousarray(ctr, dtype=np.uint64)
    k = np.ascontiguousarray(key, dtype=np.uint64)
    out = np.empty(4, dtype=np.uint64)
    lib().cpvo_philox4x64(_p(c), _p(k), _p(out))
    return out


def philox_uniforms(seed, B, k, round=0):
    """u[b][j][r] from Philox4x64-10, counter (b, j, r, round), key (seed, 0)."""
    u = np.empty((B, k + 1, 2), dtype=np.float32)
    lib().cpvo_philox_uniforms(seed, round, B, k, _p(u))
    return u


class Rng:
    """xoshiro256++ (crates/codpiece-sample/src/lib.rs:88-130)."""

    def __init__(self, seed):
        self.s = np.zeros(4, dtype=np.uint64)
        lib().cpvo_rng_seed(seed, _p(self.s))

    def next_u64(self):
        return lib().cpvo_rng_next_u64(_p(self.s))

    def next_f32(self):
        return lib().cpvo_rng_next_f32(_p(self.s))


def row_bytes(t, k):
    assert k % BLOCK[t] == 0
    return k // BLOCK[t] * SIZE[t]


def quantize(t, x):
    """Quantize rows of x (last axis = K) into ggml blocks; returns uint8 [.., row_bytes]."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    k = x.shape[-1]
    out = np.empty(x.shape[:-1] + (row_bytes(t, k),), dtype=np.uint8)
    assert lib().cpvo_quantize(t, _p(x), x.size, _p(out)) == 0
    return out


def dequantize(t, q, k):
    q = np.ascontiguousarray(q, dtype=np.uint8)
    rows = q.size // row_bytes(t, k)
    out = np.empty((rows, k), dtype=np.float32)
    assert lib().cpvo_dequantize(t, _p(q), rows * k, _p(out)) == 0
    return out.reshape(q.shape[:-1] + (k,))


def qgemm(t, w, x, threads=8):
    """y[M][N] = x[M][K] . dequant(w[N][K])^T under the exact-window contract."""
    w = np.ascontiguousarray(w, dtype=np.uint8)
    x = np.ascontiguousarray(x, dtype=np.float32)
    M, K = x.shape
    N = w.size // row_bytes(t, K)
    y = np.empty((M, N), dtype=np.float32)
    assert lib().cpvo_qgemm(t, _p(w), N, K, _p(x), M, _p(y), threads) == 0
    return y


def qgemm_f64(t, w, x, threads=8):
    w = np.ascontiguousarray(w, dtype=np.uint8)
    x = np.ascontiguousarray(x, dtype=np.float32)
    M, K = x.shape
    N = w.size // row_bytes(t, K)
    y = np.empty((M, N), dtype=np.float64)
    assert lib().cpvo_qgemm_f64(t, _p(w), N, K, _p(x), M, _p(y), threads) == 0
    return y


def mul_mat_f32(w, x):
    w = np.ascontiguousarray(w, dtype=np.float32)
    x = np.ascontiguousarray(x, dtype=np.float32)
    N, K = w.shape
    M = x.shape[0]
    y = np.empty((M, N), dtype=np.float32)
    lib().cpvo_mul_mat_f32(_p(w), N, K, _p(x), M, _p(y))
    return y


def rms_norm(x, eps, w=None):
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty_like(x)
    n = x.shape[-1]
    wa = None if w is None else np.ascontiguousarray(w, dtype=np.float32)
    for r in range(x.size // n):
        xr = x.reshape(-1, n)[r]
        orow = out.reshape(-1, n)[r]
        lib().cpvo_rms_norm(_p(xr), n, eps, _p(wa), _p(orow))
    return out


def rope_table(n_pos, n_rot, freq_base, sections=None):
    cs = np.empty((n_pos, n_rot // 2, 2), dtype=np.float32)
    if sections is None:
        lib().cpvo_rope_table(n_pos, n_rot, freq_base, _p(cs))
    else:
        s = np.ascontiguousarray(sections, dtype=np.int32)
        lib().cpvo_rope_table_sections(n_pos, n_rot, freq_base, _p(s), _p(cs))
    return cs


def rope_neox(x, n_rot, cs_row):
    x = np.array(x, dtype=np.float32, copy=True)
    cs_row = np.ascontiguousarray(cs_row, dtype=np.float32)
    lib().cpvo_rope_neox(_p(x), n_rot, _p(cs_row))
    return x


ATTN_CHUNK = 128


def attn(q, kc, vc, n_past, parent, scale, f64=False):
    """q [T][H][D] f32; kc/vc [n_ctx][Hkv*D] uint16 (f16 bits).  The
    exact-window contract, or (f64=True) binary64 attention."""
    q = np.ascontiguousarray(q, dtype=np.float32)
    T, H, D = q.shape
    kc = np.ascontiguousarray(kc, dtype=np.uint16)
    vc = np.ascontiguousarray(vc, dtype=np.uint16)
    Hkv = kc.shape[1] // D
    par = None if parent is None else np.ascontiguousarray(parent, dtype=np.int32)
    out = np.empty((T, H * D), dtype=np.float32)
    fn = lib().cpvo_attn_f64 if f64 else lib().cpvo_attn
    fn(_p(q), _p(kc), _p(vc), n_past, _p(par), T, H, Hkv, D, scale, _p(out))
    return out


def distribution(params, logits, hist=None):
    logits = np.ascontiguousarray(logits, dtype=np.float32)
    V = logits.size
    h = None if hist is None or len(hist) == 0 else np.ascontiguousarray(hist, dtype=np.int32)
    ids = np.empty(V, dtype=np.int32)
    probs = np.empty(V, dtype=np.float32)
    tl = np.empty(V, dtype=np.float32)
    n = lib().cpvo_distribution(ctypes.byref(params), _p(logits), V, _p(h),
                                0 if h is None else h.size, _p(ids), _p(probs), _p(tl))
    return ids[:n].copy(), probs[:n].copy(), tl[:n].copy()


class Dist:
    """Mirror of Dist (crates/codpiece-sample/src/lib.rs:378-451)."""

    def __init__(self, ids, probs):
        self.ids = np.ascontiguousarray(ids, dtype=np.int32)
        self.probs = np.ascontiguousarray(probs, dtype=np.float32)

    def __len__(self):
        return self.ids.size

    def prob_of(self, tok):
        return lib().cpvo_dist_prob_of(_p(self.ids), _p(self.probs), self.ids.size, tok)

    def draw(self, r):
        return lib().cpvo_dist_draw(_p(self.ids), _p(self.probs), self.ids.size, r)

    def draw_excluding(self, tok, r):
        return lib().cpvo_dist_draw_excluding(_p(self.ids), _p(self.probs), self.ids.size, tok, r)

    def peak(self):
        return lib().cpvo_dist_peak(_p(self.probs), self.ids.size)


class Sampler:
    """Mirror of Sampler (crates/codpiece-sample/src/lib.rs:132-227)."""

    def __init__(self, params, seed=0):
        self.params = params
        self.rng = Rng(seed)
        self.history = []

    def accept(self, tok):
        if self.params.penalty_last_n == 0:
            return
        self.history.append(tok)
        while len(self.history) > self.params.penalty_last_n:
            self.history.pop(0)

    def distribution(self, logits):
        ids, probs, _ = distribution(self.params, logits, self.history)
        return Dist(ids, probs)

    def sample(self, logits):
        d = self.distribution(logits)
        return d.draw(self.rng.next_f32())

    def sample_coupled(self, logits, noise_t):
        logits = np.ascontiguousarray(logits, dtype=np.float32)
        noise_t = np.ascontiguousarray(noise_t, dtype=np.float32)
        h = None if not self.history else np.asarray(self.history, dtype=np.int32)
        return lib().cpvo_sample_coupled(ctypes.byref(self.params), _p(logits), logits.size,
                                         _p(h), 0 if h is None else h.size, _p(noise_t))


def argmax(x):
    x = np.ascontiguousarray(x, dtype=np.float32)
    return lib().cpvo_argmax(_p(x), x.size)


def softmax_peak_seq(x):
    """1 / (index-order f32 sum of exp(x - max)): the re-draft gate's value
    (engine.rs:2598-2606)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    return float(lib().cpvo_softmax_peak_seq(_p(x), x.size))


def spec_accept(p_logits, draft, params, mode, u=None, q_logits=None, noise_t=None, hist=None):
    """Acceptance for B sequences: returns (tokens [B][k+1], n_accept [B])."""
    p_logits = np.ascontiguousarray(p_logits, dtype=np.float32)
    B, k1, V = p_logits.shape
    k = k1 - 1
    draft = np.ascontiguousarray(draft, dtype=np.int32).reshape(B, k)
    q = None if q_logits is None else np.ascontiguousarray(q_logits, dtype=np.float32)
    uu = None if u is None else np.ascontiguousarray(u, dtype=np.float32)
    nz = None if noise_t is None else np.ascontiguousarray(noise_t, dtype=np.float32)
    h = None if hist is None else np.ascontiguousarray(hist, dtype=np.int32)
    hl = 0 if h is None else h.shape[1]
    tok = np.full((B, k + 1), -1, dtype=np.int32)
    n = np.empty(B, dtype=np.int32)
    lib().cpvo_spec_accept(_p(p_logits), _p(q), _p(draft), B, k, V, ctypes.byref(params), mode,
                           _p(uu), _p(nz), _p(h), hl, _p(tok), _p(n))
    return tok, n


def spec_accept_rng(p_logits, draft, params, rng, hist=None):
    """The engine loop with the reference's sequential RNG; returns
    (tokens, n_accept, uniforms used by role [k+1][2])."""
    p_logits = np.ascontiguousarray(p_logits, dtype=np.float32)
    k1, V = p_logits.shape
    k = k1 - 1
    draft = np.ascontiguousarray(draft, dtype=np.int32)
    h = None if not hist else np.asarray(hist, dtype=np.int32)
    tok = np.full(k + 1, -1, dtype=np.int32)
    used = np.empty((k + 1, 2), dtype=np.float32)
    n = lib().cpvo_spec_accept_rng(_p(p_logits), _p(draft), k, V, ctypes.byref(params),
                                   _p(rng.s), _p(h), 0 if h is None else h.size, _p(tok), _p(used))
    return tok, n, used


def set_fault(code):
    """Plant one of the oracle's listed composition mistakes (cpvo.h), or 0."""
    lib().cpvo_set_fault(int(code))


def set_attn_f64(on):
    """Run the model round's attention in binary64 instead of the contract."""
    lib().cpvo_set_attn_f64(1 if on else 0)


def set_smooth(on):
    """Run the model round's mul_mats on unquantized activations (binary64 sums)."""
    lib().cpvo_set_smooth(1 if on else 0)


def set_threads(n):
    """Threads of the model round's GEMMs and attention."""
    lib().cpvo_set_threads(int(n))


class Hparams(ctypes.Structure):
    _fields_ = [
        ("n_layer", ctypes.c_int32), ("n_embd", ctypes.c_int32), ("n_head", ctypes.c_int32),
        ("n_head_kv", ctypes.c_int32), ("head_dim", ctypes.c_int32), ("n_ff", ctypes.c_int32),
        ("n_vocab", ctypes.c_int32), ("n_rot", ctypes.c_int32), ("rope_sections", ctypes.c_int32 * 4),
        ("rms_eps", ctypes.c_float), ("freq_base", ctypes.c_float), ("has_mtp", ctypes.c_int32),
    ]


class Model:
    """The oracle's restatement of the qwen35 verify round (cpvo_model.c)."""

    def __init__(self, hp_fields):
        self.hp = Hparams()
        for k, v in hp_fields.items():
            if k == "rope_sections":
                for i, x in enumerate(v):
                    self.hp.rope_sections[i] = x
            else:
                setattr(self.hp, k, v)
        self.h = lib().cpvo_model_create(ctypes.byref(self.hp))

    def set_tensor(self, name, qtype, data, ne0, ne1):
        data = np.ascontiguousarray(data)
        assert lib().cpvo_model_set(self.h, name.encode(), qtype, _p(data), ne0, ne1) == 0, name

    def free(self):
        if self.h:
            lib().cpvo_model_free(self.h)
            self.h = None


class Session:
    def __init__(self, model, n_ctx):
        self.model = model
        self.h = lib().cpvo_session_create(model.h, n_ctx)

    @property
    def pos(self):
        a, b = np.zeros(1, np.int64), np.zeros(1, np.int64)
        lib().cpvo_session_get_pos(self.h, _p(a), _p(b))
        return int(a[0]), int(b[0])

    def set_pos(self, n_past, mtp_past):
        lib().cpvo_session_set_pos(self.h, n_past, mtp_past)

    def inject_attention(self, att):
        """Continue the next call with these attention outputs (float32 blocks
        in call order, or None); returns nothing, see inject_ratio."""
        self._inj = None if att is None else np.ascontiguousarray(att, dtype=np.float32).ravel()
        lib().cpvo_session_set_attn_inject(self.h, _p(self._inj), 0 if att is None else self._inj.size)

    @property
    def inject_ratio(self):
        return lib().cpvo_session_inject_ratio(self.h)

    def prefill(self, tokens):
        t = np.ascontiguousarray(tokens, dtype=np.int32)
        assert lib().cpvo_prefill(self.h, _p(t), t.size) == 0

    def step_fused_cached(self, tokens, depth, want_logits=False, noise=None, cands=None):
        t = np.ascontiguousarray(tokens, dtype=np.int32)
        T, V, E = t.size, self.model.hp.n_vocab, self.model.hp.n_embd
        preds = np.empty(T, np.int32)
        chain = np.empty((max(depth, 1), T), np.int32)
        conf = np.empty((max(depth, 1), T), np.float32)
        logits = np.empty((T, V), np.float32) if want_logits else None
        hidden = np.empty((T, E), np.float32) if want_logits else None
        nz = None if noise is None else np.ascontiguousarray(noise, dtype=np.float32)
        c = None if cands is None else np.ascontiguousarray(cands, dtype=np.int32)
        assert lib().cpvo_verify_step_cands(self.h, _p(t), T, depth, _p(nz), _p(c), 0 if c is None else c.size,
                                            _p(preds), _p(chain), _p(conf), _p(logits), _p(hidden)) == 0
        return preds, chain[:depth], conf[:depth], logits, hidden

    def mtp_draft(self, hidden, token, pos):
        """One standalone draft link (Qwen35::mtp_draft): (logits [V], hidden
        [E]); mtp_past advances by 1."""
        V, E = self.model.hp.n_vocab, self.model.hp.n_embd
        h = np.ascontiguousarray(hidden, dtype=np.float32).ravel()
        assert h.size == E
        logits, hout = np.empty(V, np.float32), np.empty(E, np.float32)
        assert lib().cpvo_mtp_draft(self.h, _p(h), int(token), int(pos), _p(logits), _p(hout)) == 0
        return logits, hout

    def fused_generate(self, prompt, n_gen, depth, tail=64, bulk=512):
        p = np.ascontiguousarray(prompt, dtype=np.int32)
        out = np.empty(n_gen, np.int32)
        stats = np.zeros(3, np.int64)
        n = lib().cpvo_fused_generate(self.h, _p(p), p.size, n_gen, depth, tail, bulk, _p(out), _p(stats))
        assert n >= 0
        return out[:n].tolist(), stats.tolist()

    def free(self):
        if self.h:
            lib().cpvo_session_free(self.h)
            self.h = None
