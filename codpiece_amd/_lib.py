"""ctypes binding of libcpv.so — the C ABI declared in include/cpv.h.

This is the binding a host maintainer would write over the library; it loads the
in-tree build and fails loudly when it is missing.  There is no fallback path:
every compute call goes through the HIP library.
"""
import ctypes
import os

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libcpv.so")

CPV_OK, CPV_EINVAL, CPV_ENOMEM, CPV_EDEVICE, CPV_EUNSUPPORTED = 0, 1, 2, 3, 4
F32, F16, Q8_0, Q4_K, Q6_K = 0, 1, 8, 12, 14
ACCEPT_GREEDY, ACCEPT_REJECT, ACCEPT_GUMBEL = 0, 1, 2

STATUS_NAMES = {0: "CPV_OK", 1: "CPV_EINVAL", 2: "CPV_ENOMEM", 3: "CPV_EDEVICE", 4: "CPV_EUNSUPPORTED"}


class CpvError(RuntimeError):
    def __init__(self, status, msg):
        super().__init__(f"{STATUS_NAMES.get(status, status)}: {msg}")
        self.status = status


class SamplerParams(ctypes.Structure):
    """cpv_sampler_params: SamplerParams of crates/codpiece-sample/src/lib.rs:29-64
    without the seed (uniforms are explicit)."""
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
                 penalty_repeat=1.0, penalty_freq=0.0, penalty_present=0.0, penalty_last_n=64):
        super().__init__(temp, top_k, top_p, min_p, min_keep, penalty_repeat, penalty_freq,
                         penalty_present, penalty_last_n)


class Hparams(ctypes.Structure):
    """cpv_hparams: an all-attention qwen35 model (crates/codpiece-model/src/qwen35.rs:45-148)."""
    _fields_ = [
        ("n_layer", ctypes.c_int32), ("n_embd", ctypes.c_int32), ("n_head", ctypes.c_int32),
        ("n_head_kv", ctypes.c_int32), ("head_dim", ctypes.c_int32), ("n_ff", ctypes.c_int32),
        ("n_vocab", ctypes.c_int32), ("n_rot", ctypes.c_int32), ("rope_sections", ctypes.c_int32 * 4),
        ("rms_eps", ctypes.c_float), ("freq_base", ctypes.c_float), ("has_mtp", ctypes.c_int32),
    ]


class RoundOut(ctypes.Structure):
    """cpv_round_out: FusedOut (qwen35.rs:817-828) as device pointers."""
    _fields_ = [
        ("n_past", ctypes.c_int64), ("preds_dev", ctypes.c_void_p), ("chain_dev", ctypes.c_void_p),
        ("conf_dev", ctypes.c_void_p), ("logits_dev", ctypes.c_void_p), ("hidden_dev", ctypes.c_void_p),
    ]


class DraftOut(ctypes.Structure):
    """cpv_draft_out: one standalone draft link (Qwen35::mtp_draft, qwen35.rs:2086-2192)."""
    _fields_ = [
        ("logits_dev", ctypes.c_void_p), ("hidden_dev", ctypes.c_void_p), ("draft_dev", ctypes.c_void_p),
        ("keep_dev", ctypes.c_void_p),
    ]


class GgufInfo(ctypes.Structure):
    """cpv_gguf_info: what GgufFile::open reads (crates/codpiece-gguf/src/lib.rs:345-458)."""
    _fields_ = [
        ("version", ctypes.c_int32), ("n_tensors", ctypes.c_int64), ("n_kv", ctypes.c_int64),
        ("alignment", ctypes.c_uint64), ("data_start", ctypes.c_uint64), ("tensor_bytes", ctypes.c_uint64),
    ]


(PROF_Q4_K, PROF_Q6_K, PROF_Q8_0, PROF_ATTN, PROF_SAMPLE, PROF_Q4_K_WIDE, PROF_Q8_0_WIDE, PROF_Q6_K_WIDE,
 PROF_CLASSES) = range(9)
PROF_NAMES = ("qgemm_q4_k", "qgemm_q6_k", "qgemm_q8_0", "attention", "sampler", "qgemm_q4_k_wide", "qgemm_q8_0_wide",
              "qgemm_q6_k_wide")


class ProfStat(ctypes.Structure):
    _fields_ = [("launches", ctypes.c_int64), ("ms", ctypes.c_double), ("bytes", ctypes.c_double)]


_P = ctypes.c_void_p
_I64 = ctypes.c_int64
_I32 = ctypes.c_int32
_INT = ctypes.c_int
_F32 = ctypes.c_float

# name -> (restype, argtypes); kept in the order of include/cpv.h
SIGNATURES = {
    "cpv_init": (_INT, [_INT, ctypes.POINTER(_P)]),
    "cpv_free": (None, [_P]),
    "cpv_last_error": (ctypes.c_char_p, [_P]),
    "cpv_set_stream": (_INT, [_P, _P]),
    "cpv_get_stream": (_P, [_P]),
    "cpv_profile_start": (_INT, [_P]),
    "cpv_profile_stop": (_INT, [_P, _P]),
    "cpv_profile_replay": (_INT, [_P, _INT, _INT, ctypes.POINTER(ctypes.c_double), ctypes.POINTER(ctypes.c_double)]),
    "cpv_sync": (_INT, [_P]),
    "cpv_weight_upload": (_INT, [_P, _INT, _P, _I64, _I64, ctypes.POINTER(_P)]),
    "cpv_weight_from_device": (_INT, [_P, _INT, _P, _I64, _I64, ctypes.POINTER(_P)]),
    "cpv_weight_free": (None, [_P]),
    "cpv_weight_info": (_INT, [_P, ctypes.POINTER(_INT), ctypes.POINTER(_I64), ctypes.POINTER(_I64),
                               ctypes.POINTER(_I64)]),
    "cpv_get_rows": (_INT, [_P, _P, _P, _I64, _P]),
    "cpv_qgemm": (_INT, [_P, _P, _P, _I64, _P]),
    "cpv_qgemm_noalloc": (_INT, [_P, _P, _P, _I64, _P]),
    "cpv_attn": (_INT, [_P, _P, _P, _P, _I64, _I64, _P, _INT, _INT, _INT, _INT, _F32, _P]),
    "cpv_argmax_rows": (_INT, [_P, _P, _P, _I64, _I64, _P]),
    "cpv_distribution": (_INT, [_P, _P, _INT, _INT, ctypes.POINTER(SamplerParams), _P, _INT, _P, _P, _P]),
    "cpv_spec_accept": (_INT, [_P, _P, _P, _P, _INT, _INT, _INT, ctypes.POINTER(SamplerParams), _INT,
                               _P, ctypes.c_uint64, ctypes.c_uint64, _P, _P, _INT, _P, _P]),
    "cpv_model_create": (_INT, [_P, ctypes.POINTER(Hparams), ctypes.POINTER(_P)]),
    "cpv_model_set_tensor": (_INT, [_P, ctypes.c_char_p, _INT, _P, _INT, _I64, _I64]),
    "cpv_model_ready": (_INT, [_P]),
    "cpv_model_free": (None, [_P]),
    "cpv_gguf_scan": (_INT, [ctypes.c_char_p, ctypes.POINTER(GgufInfo), ctypes.c_char_p, _INT]),
    "cpv_gguf_hparams": (_INT, [ctypes.c_char_p, ctypes.POINTER(Hparams), ctypes.c_char_p, _INT]),
    "cpv_model_load_gguf": (_INT, [_P, ctypes.c_char_p, ctypes.POINTER(_P)]),
    "cpv_session_create": (_INT, [_P, _I64, _I32, ctypes.POINTER(_P)]),
    "cpv_session_free": (None, [_P]),
    "cpv_session_set_pos": (_INT, [_P, _I64, _I64]),
    "cpv_session_get_pos": (_INT, [_P, ctypes.POINTER(_I64), ctypes.POINTER(_I64)]),
    "cpv_session_set_attn_tap": (_INT, [_P, _P, _I64]),
    "cpv_session_set_replay": (_INT, [_P, _INT]),
    "cpv_session_replay_stats": (_INT, [_P, ctypes.POINTER(ctypes.c_int64), ctypes.POINTER(ctypes.c_int64)]),
    "cpv_prefill": (_INT, [_P, _P, _INT]),
    "cpv_verify_step": (_INT, [_P, _P, _INT, _INT, _P, ctypes.POINTER(RoundOut)]),
    "cpv_verify_step_cands": (_INT, [_P, _P, _INT, _INT, _P, ctypes.POINTER(ctypes.c_int32), _INT,
                                     ctypes.POINTER(RoundOut)]),
    "cpv_mtp_draft": (_INT, [_P, _P, _I32, _I64, _F32, ctypes.POINTER(DraftOut)]),
    "cpv_redraft_gate": (_INT, [_P, _P, _I64, _I64, _F32, _P, _P]),
    "cpv_verify_tree": (_INT, [_P, _P, ctypes.POINTER(ctypes.c_int32), _INT, _P, ctypes.POINTER(RoundOut)]),
    "cpv_session_commit_branch": (_INT, [_P, ctypes.POINTER(ctypes.c_int32), _INT]),
}

_lib = None


def load():
    """Load libcpv.so and bind every entry point; raises if it is not built."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise RuntimeError(f"{LIB_PATH} is not built; run __graft_entry__.build() "
                           "or python codpiece_amd/build.py")
    lib = ctypes.CDLL(LIB_PATH)
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _lib = lib
    return lib
