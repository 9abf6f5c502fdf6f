"""Python bindings of libsjk.so (the MI355X SJ-KVaRN codec library) over ctypes.

The library's C ABI is declared in include/sjk.h: the sj_kvarn.h API (reference sj_kvarn.h:177-453) plus
the sjk_hip_* device entry points. Device memory for the device entry points comes from the HIP runtime
itself (Device below), so no framework is needed to drive the kernels. Loading fails loudly when the
library has not been built: there is no fallback.
"""
import ctypes as C
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libsjk.so")

u8p = C.POINTER(C.c_uint8)
u16p = C.POINTER(C.c_uint16)
u32p = C.POINTER(C.c_uint32)
f32p = C.POINTER(C.c_float)
vp = C.c_void_p

BODY_SCALAR, BODY_TRELLIS, BODY_AUTO = 0, 1, 2
STAGING_TQ6, STAGING_F16 = 0, 1
SINK_F16, SINK_INHERIT = 0, 1
NO_POS = NO_BLOCK = 0xFFFFFFFF
OK, ERR_ARG, ERR_PENDING, ERR_CORRUPT, ERR_POOL_FULL = 0, -100, -108, -107, -110


class Layout(C.Structure):
    _fields_ = [("D", C.c_int), ("G", C.c_int), ("bits_k", C.c_int), ("bits_v", C.c_int), ("body", C.c_int),
                ("k_payload", C.c_uint32), ("v_payload", C.c_uint32), ("k_scale", C.c_uint32),
                ("k_zero", C.c_uint32), ("k_tok", C.c_uint32), ("v_ch", C.c_uint32), ("v_scale", C.c_uint32),
                ("v_zero", C.c_uint32), ("bytes", C.c_uint32)]


class Policy(C.Structure):
    _fields_ = [("sink", C.c_uint32), ("tail", C.c_uint32), ("tail_max", C.c_uint32), ("group", C.c_uint32),
                ("flush_chunk", C.c_uint32), ("B", C.c_uint32), ("B_prev", C.c_uint32),
                ("B_pending", C.c_uint32), ("draining", C.c_int)]


class Config(C.Structure):
    _fields_ = [("head_dim", C.c_int), ("n_head_kv", C.c_int), ("group", C.c_int), ("bits_k", C.c_int),
                ("bits_v", C.c_int), ("body", C.c_int), ("iters", C.c_int), ("staging", C.c_int),
                ("sink_type", C.c_int), ("sink", C.c_uint32), ("tail", C.c_uint32), ("tail_max", C.c_uint32),
                ("flush_chunk", C.c_uint32), ("n_ubatch", C.c_uint32), ("n_ctx", C.c_uint32)]


class Layer(C.Structure):
    _fields_ = [("cfg", Config), ("lay", Layout), ("cap", C.c_uint32), ("n_groups", C.c_uint32),
                ("stage_bytes", C.c_size_t), ("ring", vp), ("sink", vp), ("body", vp), ("work", vp),
                ("kstage", vp), ("vstage", vp), ("blocks", u32p), ("owns_body", C.c_int)]


class Pool(C.Structure):
    _fields_ = [("cfg", Config), ("lay", Layout), ("n_layers", C.c_int), ("n_blocks", C.c_uint32), ("body", vp),
                ("free_ids", u32p), ("n_free", C.c_uint32)]


class Seq(C.Structure):
    _fields_ = [("cfg", Config), ("n_layers", C.c_int), ("layers", C.POINTER(Layer)), ("pol", Policy),
                ("n", C.c_uint32), ("pool", C.POINTER(Pool)), ("blocks", u32p)]


class StateInfo(C.Structure):
    _fields_ = [("state_version", C.c_uint32), ("format_version", C.c_uint32), ("cfg", Config),
                ("rotation", C.c_uint32), ("rotation_n", C.c_uint32), ("codebook_id", C.c_uint64),
                ("n_layers", C.c_int), ("n", C.c_uint32), ("B", C.c_uint32), ("B_prev", C.c_uint32),
                ("draining", C.c_uint32), ("total_bytes", C.c_size_t)]


class View(C.Structure):
    _fields_ = [("lay", Layout), ("n_head_kv", C.c_int), ("staging", C.c_int), ("sink_type", C.c_int),
                ("S", C.c_uint32), ("cap", C.c_uint32), ("stage_bytes", C.c_size_t), ("sink", vp), ("ring", vp),
                ("body", vp), ("blocks", vp), ("work", vp), ("work_bytes", C.c_size_t)]


class AttendJob(C.Structure):
    _fields_ = [("v", View), ("B", C.c_uint32), ("N", C.c_uint32), ("qpos0", C.c_uint32), ("d_q", vp), ("d_out", vp)]


class StoreJob(C.Structure):
    _fields_ = [("v", View), ("pos0", C.c_uint32), ("d_k", vp), ("d_v", vp)]


class SeqJob(C.Structure):
    _fields_ = [("seq", C.POINTER(Seq)), ("pos0", C.c_uint32), ("d_k", vp), ("d_v", vp), ("d_q", vp), ("d_out", vp)]


LP, CP, PP, LYP, PLP, SQP = (C.POINTER(Layout), C.POINTER(Config), C.POINTER(Policy), C.POINTER(Layer),
                             C.POINTER(Pool), C.POINTER(Seq))

# every symbol include/sjk.h declares: name -> (restype, argtypes)
SIGNATURES = {
    "sj_kvarn_f32_to_f16": (C.c_uint16, [C.c_float]),
    "sj_kvarn_f16_to_f32": (C.c_float, [C.c_uint16]),
    "sj_kvarn_hadamard": (None, [f32p, C.c_int]),
    "sj_kvarn_rotate_heads": (None, [f32p, C.c_int, C.c_int]),
    "sj_kvarn_body_resolve": (C.c_int, [C.c_int, C.c_int, C.c_int]),
    "sj_kvarn_layout_init": (C.c_int, [LP, C.c_int, C.c_int, C.c_int, C.c_int, C.c_int]),
    "sj_kvarn_record_bytes": (C.c_size_t, [C.c_int, C.c_int, C.c_int, C.c_int]),
    "sj_kvarn_body_bits_per_element": (C.c_double, [LP]),
    "sj_kvarn_code_bit": (C.c_uint32, [LP, C.c_int, C.c_int, C.c_int]),
    "sj_kvarn_k_ch_idx": (C.c_int, [LP, C.c_int]),
    "sj_kvarn_v_ch_idx": (C.c_int, [LP, C.c_int]),
    "sj_kvarn_seal_workspace_bytes": (C.c_size_t, [LP]),
    "sj_kvarn_seal_group": (None, [LP, u16p, u16p, C.c_size_t, C.c_int, u8p, vp]),
    "sj_kvarn_decode_k_row": (None, [LP, u8p, C.c_int, f32p]),
    "sj_kvarn_decode_v_row": (None, [LP, u8p, C.c_int, f32p]),
    "sj_kvarn_tq6_quantize_row": (None, [f32p, vp, C.c_int]),
    "sj_kvarn_tq6_dequantize_row": (None, [vp, f32p, C.c_int]),
    "sj_kvarn_stage_row_bytes": (C.c_size_t, [C.c_int, C.c_int]),
    "sj_kvarn_stage_row": (None, [C.c_int, f32p, vp, C.c_int]),
    "sj_kvarn_unstage_row": (None, [C.c_int, vp, f32p, C.c_int]),
    "sj_kvarn_record_scores": (None, [LP, u8p, f32p, C.c_int, f32p]),
    "sj_kvarn_record_accum_v": (None, [LP, u8p, f32p, C.c_int, f32p]),
    "sj_kvarn_policy_init": (None, [PP] + [C.c_uint32] * 5),
    "sj_kvarn_policy_reset": (None, [PP]),
    "sj_kvarn_policy_begin_ubatch": (C.c_uint32, [PP, C.c_uint32, C.c_uint32]),
    "sj_kvarn_policy_commit": (None, [PP]),
    "sj_kvarn_policy_idle": (C.c_uint32, [PP, C.c_uint32, C.c_uint32]),
    "sj_kvarn_group_floor": (C.c_uint32, [C.c_uint32, C.c_uint32, C.c_uint32]),
    "sj_kvarn_policy_trunc_floor": (C.c_uint32, [PP, C.c_uint32]),
    "sj_kvarn_policy_truncate": (C.c_uint32, [PP, C.c_uint32, u32p]),
    "sj_kvarn_ring_capacity": (C.c_uint32, [C.c_uint32] * 4),
    "sj_kvarn_ring_slot": (C.c_uint32, [C.c_uint32] * 3),
    "sj_kvarn_config_default": (Config, [C.c_int, C.c_int, C.c_uint32, C.c_uint32]),
    "sj_kvarn_layer_init": (C.c_int, [LYP, CP]),
    "sj_kvarn_layer_free": (None, [LYP]),
    "sj_kvarn_layer_store": (None, [LYP, C.c_uint32, f32p, f32p]),
    "sj_kvarn_layer_seal": (None, [LYP, C.c_uint32, C.c_uint32]),
    "sj_kvarn_layer_kv_row": (None, [LYP, C.c_uint32, C.c_uint32, C.c_int, f32p, f32p]),
    "sj_kvarn_layer_attend_row": (None, [LYP, C.c_uint32, C.c_uint32, f32p, C.c_int, C.c_uint32, C.c_float, f32p]),
    "sj_kvarn_layer_record": (vp, [LYP, C.c_uint32, C.c_int]),
    "sj_kvarn_layer_truncate": (None, [LYP, C.c_uint32, C.c_uint32, C.c_uint32, C.c_uint32]),
    "sj_kvarn_strerror": (C.c_char_p, [C.c_int]),
    "sj_kvarn_pool_init": (C.c_int, [PLP, CP, C.c_int, C.c_uint32]),
    "sj_kvarn_pool_free": (None, [PLP]),
    "sj_kvarn_pool_alloc": (C.c_uint32, [PLP]),
    "sj_kvarn_pool_release": (None, [PLP, C.c_uint32]),
    "sj_kvarn_seq_init": (C.c_int, [SQP, CP, C.c_int, PLP]),
    "sj_kvarn_seq_free": (None, [SQP]),
    "sj_kvarn_seq_reset": (None, [SQP]),
    "sj_kvarn_seq_begin_ubatch": (C.c_int, [SQP, C.c_uint32, C.c_uint32]),
    "sj_kvarn_seq_store": (None, [SQP, C.c_uint32, f32p, f32p]),
    "sj_kvarn_seq_idle": (C.c_int, [SQP, C.c_uint32]),
    "sj_kvarn_seq_truncate": (C.c_uint32, [SQP, C.c_uint32]),
    "sj_kvarn_seq_attend_row": (None, [SQP, C.c_int, f32p, C.c_int, C.c_uint32, C.c_float, f32p]),
    "sj_kvarn_seq_state_size": (C.c_size_t, [SQP]),
    "sj_kvarn_state_size_max": (C.c_size_t, [CP, C.c_int]),
    "sj_kvarn_seq_state_write": (C.c_int, [SQP, vp, C.c_size_t, C.POINTER(C.c_size_t)]),
    "sj_kvarn_state_peek": (C.c_int, [vp, C.c_size_t, C.POINTER(StateInfo)]),
    "sj_kvarn_seq_state_read": (C.c_int, [SQP, vp, C.c_size_t]),
    "sjk_hip_supported": (C.c_int, [LP]),
    "sjk_hip_workspace_bytes": (C.c_size_t, [LP, C.c_int]),
    "sjk_hip_seal": (C.c_int, [LP, vp, vp, C.c_size_t, C.c_int, C.c_int, C.c_int, vp, vp]),
    "sjk_hip_decode": (C.c_int, [LP, vp, C.c_int, vp, vp, vp]),
    "sjk_hip_stage": (C.c_int, [C.c_int, vp, vp, C.c_int, C.c_size_t, C.c_int, vp]),
    "sjk_hip_unstage": (C.c_int, [C.c_int, vp, C.c_size_t, vp, C.c_int, C.c_int, vp]),
    "sjk_hip_rotate": (C.c_int, [vp, C.c_int, C.c_int, vp]),
    "sjk_hip_fold_rotation_out": (C.c_int, [vp, C.c_int, C.c_int, C.c_int, vp]),
    "sjk_hip_fold_rotation_in": (C.c_int, [vp, C.c_int, C.c_int, C.c_int, vp]),
    "sjk_hip_layer_store": (C.c_int, [C.POINTER(View), C.c_uint32, C.c_uint32, vp, vp, C.c_int, vp]),
    "sjk_hip_commit": (C.c_int, [C.POINTER(View), C.c_int, C.c_uint32, C.c_uint32, C.c_int, vp]),
    "sjk_hip_commit_dyn": (C.c_int, [C.POINTER(View), C.c_int, vp, C.c_int, C.c_int, vp]),
    "sjk_hip_attend_dyn": (C.c_int, [C.POINTER(View), vp, C.c_uint32, C.c_int, C.c_int, vp, C.c_float, vp, vp]),
    "sjk_hip_layer_store_dyn": (C.c_int, [C.POINTER(View), vp, C.c_uint32, vp, vp, C.c_int, vp]),
    "sjk_hip_attend": (C.c_int, [C.POINTER(View), C.c_uint32, C.c_uint32, C.c_uint32, C.c_int, C.c_int, vp,
                                 C.c_float, vp, vp]),
    "sjk_hip_attend_noalloc": (C.c_int, [C.POINTER(View), C.c_uint32, C.c_uint32, C.c_uint32, C.c_int, C.c_int, vp,
                                         C.c_float, vp, vp]),
    "sjk_hip_kv_rows": (C.c_int, [C.POINTER(View), C.c_uint32, C.c_uint32, C.c_uint32, C.c_int, vp, vp, vp]),
    "sjk_hip_record_scores": (C.c_int, [LP, vp, vp, C.c_int, vp, vp]),
    "sjk_hip_record_accum_v": (C.c_int, [LP, vp, vp, C.c_int, vp, vp]),
    "sjk_hip_seq_store": (C.c_int, [SQP, C.c_int, C.c_uint32, C.c_uint32, vp, vp, C.c_int, vp]),
    "sjk_hip_seq_attend": (C.c_int, [SQP, C.c_int, C.c_uint32, C.c_int, C.c_int, vp, C.c_float, vp, vp]),
    "sjk_hip_attend_batch": (C.c_int, [C.POINTER(AttendJob), C.c_int, C.c_int, C.c_int, C.c_float, vp]),
    "sjk_hip_store_batch": (C.c_int, [C.POINTER(StoreJob), C.c_int, C.c_uint32, C.c_int, vp]),
    "sjk_hip_seq_store_batch": (C.c_int, [C.POINTER(SeqJob), C.c_int, C.c_int, C.c_uint32, C.c_int, vp]),
    "sjk_hip_seq_begin_ubatch": (C.c_int, [SQP, C.c_uint32, C.c_uint32, vp]),
    "sjk_hip_seq_idle": (C.c_int, [SQP, C.c_uint32, vp]),
    "sjk_hip_seq_state_write_begin": (C.c_int, [SQP, vp, C.c_size_t]),
    "sjk_hip_seq_state_read_begin": (C.c_int, [SQP, vp, C.c_size_t]),
    "sjk_hip_seq_state_poll": (C.c_int, [SQP]),
    "sjk_hip_seq_state_finish": (C.c_int, [SQP, C.POINTER(C.c_size_t)]),
    "sjk_hip_seq_attend_batch": (C.c_int, [C.POINTER(SeqJob), C.c_int, C.c_int, C.c_int, C.c_int, C.c_float, vp]),
    "sjk_hip_balance_step": (C.c_int, [vp, vp, vp, C.c_int, vp]),
    "sjk_layer_view": (View, [LYP]),
    "sjk_last_error": (C.c_char_p, []),
}

_lib = None


def load(path=LIB_PATH):
    """Load libsjk.so and bind every declared symbol. Raises when the library or a symbol is missing."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(path):
        raise RuntimeError("libsjk.so is not built (%s): run __graft_entry__.build()" % path)
    lib = C.CDLL(path)
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)   # AttributeError: a declared entry point is missing
        fn.restype = res
        fn.argtypes = args
    _lib = lib
    return lib


def check(rc, what="call"):
    if rc != 0:
        lib = load()
        raise RuntimeError("%s failed: %d (%s; %s)" % (what, rc, lib.sj_kvarn_strerror(rc).decode(),
                                                      lib.sjk_last_error().decode()))


class Device:
    """Minimal device-memory helper over the HIP runtime (the library's own runtime)."""
    H2D, D2H, D2D = 1, 2, 3

    def __init__(self):
        load()
        self.hip = C.CDLL("libamdhip64.so")
        self.hip.hipMalloc.argtypes = [C.POINTER(vp), C.c_size_t]
        self.hip.hipFree.argtypes = [vp]
        self.hip.hipMemcpy.argtypes = [vp, vp, C.c_size_t, C.c_int]
        self.hip.hipMemcpyAsync.argtypes = [vp, vp, C.c_size_t, C.c_int, vp]
        self.hip.hipMemset.argtypes = [vp, C.c_int, C.c_size_t]
        self.hip.hipStreamCreate.argtypes = [C.POINTER(vp)]
        self.hip.hipStreamDestroy.argtypes = [vp]
        self.hip.hipStreamSynchronize.argtypes = [vp]
        self.hip.hipEventCreate.argtypes = [C.POINTER(vp)]
        self.hip.hipEventRecord.argtypes = [vp, vp]
        self.hip.hipEventSynchronize.argtypes = [vp]
        self.hip.hipEventElapsedTime.argtypes = [C.POINTER(C.c_float), vp, vp]
        self.hip.hipEventDestroy.argtypes = [vp]
        self.hip.hipGetErrorString.restype = C.c_char_p
        self.ptrs = []

    def _ck(self, rc, what):
        if rc != 0:
            raise RuntimeError("%s: %s" % (what, self.hip.hipGetErrorString(rc).decode()))

    def alloc(self, nbytes, zero=True):
        p = vp()
        self._ck(self.hip.hipMalloc(C.byref(p), max(int(nbytes), 1)), "hipMalloc")
        if zero:
            self._ck(self.hip.hipMemset(p, 0, max(int(nbytes), 1)), "hipMemset")
        self.ptrs.append(p)
        return p

    def put(self, arr):
        arr = np.ascontiguousarray(arr)
        p = self.alloc(arr.nbytes, zero=False)
        self._ck(self.hip.hipMemcpy(p, arr.ctypes.data, arr.nbytes, self.H2D), "hipMemcpy H2D")
        return p

    def upload(self, p, arr, offset=0):
        arr = np.ascontiguousarray(arr)
        self._ck(self.hip.hipMemcpy(vp(p.value + offset), arr.ctypes.data, arr.nbytes, self.H2D), "hipMemcpy H2D")

    def get(self, p, nbytes, dtype, offset=0):
        out = np.empty(int(nbytes) // np.dtype(dtype).itemsize, dtype)
        self._ck(self.hip.hipMemcpy(out.ctypes.data, vp(p.value + offset), out.nbytes, self.D2H), "hipMemcpy D2H")
        return out

    def sync(self):
        self._ck(self.hip.hipDeviceSynchronize(), "hipDeviceSynchronize")

    def stream(self):
        s = vp()
        self._ck(self.hip.hipStreamCreate(C.byref(s)), "hipStreamCreate")
        return s

    def event(self):
        e = vp()
        self._ck(self.hip.hipEventCreate(C.byref(e)), "hipEventCreate")
        return e

    def elapsed_ms(self, e0, e1):
        ms = C.c_float()
        self._ck(self.hip.hipEventSynchronize(e1), "hipEventSynchronize")
        self._ck(self.hip.hipEventElapsedTime(C.byref(ms), e0, e1), "hipEventElapsedTime")
        return ms.value

    def free(self, p):
        self._ck(self.hip.hipFree(p), "hipFree")
        self.ptrs = [x for x in self.ptrs if x.value != p.value]

    def free_all(self):
        for p in self.ptrs:
            self.hip.hipFree(p)
        self.ptrs = []


def layout(D, G, bits_k, bits_v, body):
    lib = load()
    lay = Layout()
    rc = lib.sj_kvarn_layout_init(C.byref(lay), D, G, bits_k, bits_v, lib.sj_kvarn_body_resolve(body, bits_k, bits_v))
    if rc:
        raise ValueError("layout_init: %d" % rc)
    return lay
