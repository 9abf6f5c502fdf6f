"""ctypes bindings shared by the tests and bench.py.

Three libraries expose the same C API shape with different symbol prefixes:
  * the product, ``sj-kvarn-codec_amd/libsjk.so`` (prefix ``sj_kvarn_``; HIP kernels underneath),
  * the CPU oracle, ``oracle/libsjo.so`` (prefix ``sjo_``; test infrastructure),
  * the reference compiled from its own header, ``oracle/_ref/libsjk_ref.so`` (prefix ``sj_kvarn_``).
The structs below follow the field order of sj_kvarn.h:170-175, 228-234, 279-309, 368-396, 434-442,
which is the ABI all three share.
"""
import ctypes as C
import os

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "sj-kvarn-codec_amd")
ORACLE_SO = os.path.join(ROOT, "oracle", "libsjo.so")
REF_SO = os.path.join(ROOT, "oracle", "_ref", "libsjk_ref.so")
PRODUCT_SO = os.path.join(PKG, "libsjk.so")

u8p = C.POINTER(C.c_uint8)
u16p = C.POINTER(C.c_uint16)
u32p = C.POINTER(C.c_uint32)
f32p = C.POINTER(C.c_float)


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
                ("stage_bytes", C.c_size_t), ("ring", u8p), ("sink", u8p), ("body", u8p), ("work", C.c_void_p),
                ("kstage", u16p), ("vstage", u16p), ("blocks", u32p), ("owns_body", C.c_int)]


class Pool(C.Structure):
    _fields_ = [("cfg", Config), ("lay", Layout), ("n_layers", C.c_int), ("n_blocks", C.c_uint32), ("body", u8p),
                ("free_ids", u32p), ("n_free", C.c_uint32)]


class Seq(C.Structure):
    _fields_ = [("cfg", Config), ("n_layers", C.c_int), ("layers", C.POINTER(Layer)), ("pol", Policy),
                ("n", C.c_uint32), ("pool", C.POINTER(Pool)), ("blocks", u32p)]


class StateInfo(C.Structure):
    _fields_ = [("state_version", C.c_uint32), ("format_version", C.c_uint32), ("cfg", Config),
                ("rotation", C.c_uint32), ("rotation_n", C.c_uint32), ("codebook_id", C.c_uint64),
                ("n_layers", C.c_int), ("n", C.c_uint32), ("B", C.c_uint32), ("B_prev", C.c_uint32),
                ("draining", C.c_uint32), ("total_bytes", C.c_size_t)]


_SIGS = {
    # name: (restype, argtypes)
    "f32_to_f16": (C.c_uint16, [C.c_float]),
    "f16_to_f32": (C.c_float, [C.c_uint16]),
    "hadamard": (None, [f32p, C.c_int]),
    "rotate_heads": (None, [f32p, C.c_int, C.c_int]),
    "body_resolve": (C.c_int, [C.c_int, C.c_int, C.c_int]),
    "layout_init": (C.c_int, [C.POINTER(Layout), C.c_int, C.c_int, C.c_int, C.c_int, C.c_int]),
    "record_bytes": (C.c_size_t, [C.c_int, C.c_int, C.c_int, C.c_int]),
    "code_bit": (C.c_uint32, [C.POINTER(Layout), C.c_int, C.c_int, C.c_int]),
    "k_ch_idx": (C.c_int, [C.POINTER(Layout), C.c_int]),
    "v_ch_idx": (C.c_int, [C.POINTER(Layout), C.c_int]),
    "seal_workspace_bytes": (C.c_size_t, [C.POINTER(Layout)]),
    "seal_group": (None, [C.POINTER(Layout), u16p, u16p, C.c_size_t, C.c_int, u8p, C.c_void_p]),
    "decode_k_row": (None, [C.POINTER(Layout), u8p, C.c_int, f32p]),
    "decode_v_row": (None, [C.POINTER(Layout), u8p, C.c_int, f32p]),
    "tq6_quantize_row": (None, [f32p, C.c_void_p, C.c_int]),
    "tq6_dequantize_row": (None, [C.c_void_p, f32p, C.c_int]),
    "stage_row_bytes": (C.c_size_t, [C.c_int, C.c_int]),
    "stage_row": (None, [C.c_int, f32p, C.c_void_p, C.c_int]),
    "unstage_row": (None, [C.c_int, C.c_void_p, f32p, C.c_int]),
    "record_scores": (None, [C.POINTER(Layout), u8p, f32p, C.c_int, f32p]),
    "record_accum_v": (None, [C.POINTER(Layout), u8p, f32p, C.c_int, f32p]),
    "policy_init": (None, [C.POINTER(Policy)] + [C.c_uint32] * 5),
    "policy_reset": (None, [C.POINTER(Policy)]),
    "policy_begin_ubatch": (C.c_uint32, [C.POINTER(Policy), C.c_uint32, C.c_uint32]),
    "policy_commit": (None, [C.POINTER(Policy)]),
    "policy_idle": (C.c_uint32, [C.POINTER(Policy), C.c_uint32, C.c_uint32]),
    "group_floor": (C.c_uint32, [C.c_uint32, C.c_uint32, C.c_uint32]),
    "policy_trunc_floor": (C.c_uint32, [C.POINTER(Policy), C.c_uint32]),
    "policy_truncate": (C.c_uint32, [C.POINTER(Policy), C.c_uint32, u32p]),
    "ring_capacity": (C.c_uint32, [C.c_uint32] * 4),
    "ring_slot": (C.c_uint32, [C.c_uint32] * 3),
    "config_default": (Config, [C.c_int, C.c_int, C.c_uint32, C.c_uint32]),
    "layer_init": (C.c_int, [C.POINTER(Layer), C.POINTER(Config)]),
    "layer_free": (None, [C.POINTER(Layer)]),
    "layer_store": (None, [C.POINTER(Layer), C.c_uint32, f32p, f32p]),
    "layer_seal": (None, [C.POINTER(Layer), C.c_uint32, C.c_uint32]),
    "layer_kv_row": (None, [C.POINTER(Layer), C.c_uint32, C.c_uint32, C.c_int, f32p, f32p]),
    "layer_attend_row": (None, [C.POINTER(Layer), C.c_uint32, C.c_uint32, f32p, C.c_int, C.c_uint32, C.c_float, f32p]),
    "layer_record": (u8p, [C.POINTER(Layer), C.c_uint32, C.c_int]),
    "layer_truncate": (None, [C.POINTER(Layer), C.c_uint32, C.c_uint32, C.c_uint32, C.c_uint32]),
    "strerror": (C.c_char_p, [C.c_int]),
    "pool_init": (C.c_int, [C.POINTER(Pool), C.POINTER(Config), C.c_int, C.c_uint32]),
    "pool_free": (None, [C.POINTER(Pool)]),
    "pool_alloc": (C.c_uint32, [C.POINTER(Pool)]),
    "pool_release": (None, [C.POINTER(Pool), C.c_uint32]),
    "seq_init": (C.c_int, [C.POINTER(Seq), C.POINTER(Config), C.c_int, C.POINTER(Pool)]),
    "seq_free": (None, [C.POINTER(Seq)]),
    "seq_reset": (None, [C.POINTER(Seq)]),
    "seq_begin_ubatch": (C.c_int, [C.POINTER(Seq), C.c_uint32, C.c_uint32]),
    "seq_store": (None, [C.POINTER(Seq), C.c_uint32, f32p, f32p]),
    "seq_idle": (C.c_int, [C.POINTER(Seq), C.c_uint32]),
    "seq_truncate": (C.c_uint32, [C.POINTER(Seq), C.c_uint32]),
    "seq_attend_row": (None, [C.POINTER(Seq), C.c_int, f32p, C.c_int, C.c_uint32, C.c_float, f32p]),
    "seq_state_size": (C.c_size_t, [C.POINTER(Seq)]),
    "state_size_max": (C.c_size_t, [C.POINTER(Config), C.c_int]),
    "seq_state_write": (C.c_int, [C.POINTER(Seq), C.c_void_p, C.c_size_t, C.POINTER(C.c_size_t)]),
    "state_peek": (C.c_int, [C.c_void_p, C.c_size_t, C.POINTER(StateInfo)]),
    "seq_state_read": (C.c_int, [C.POINTER(Seq), C.c_void_p, C.c_size_t]),
}

_ORACLE_EXTRA = {
    "fnv1a": (C.c_uint64, [C.c_void_p, C.c_size_t, C.c_uint64]),
    "vec_fill_group": (None, [C.c_int, C.c_int, C.c_uint32, u16p, u16p]),
    "vec_fill_rows": (None, [C.c_int, C.c_int, f32p]),
    "st_val": (C.c_float, [C.c_uint32, C.c_uint32, C.c_uint32, C.c_uint32, C.c_int]),
    "balance_step": (None, [f32p, C.POINTER(C.c_double), f32p, C.c_size_t]),
    "st_grow": (C.c_int, [C.POINTER(Seq), C.c_uint32, C.c_uint32, C.c_uint32, C.c_uint32, C.c_uint32, C.c_uint32]),
}


class Api:
    """Binds the common API of one library under short names (api.seal_group, api.layout_init, ...)."""

    def __init__(self, path, prefix, extra=None):
        self.path = path
        self.lib = C.CDLL(path)
        self.prefix = prefix
        sigs = dict(_SIGS)
        if extra:
            sigs.update(extra)
        for name, (res, args) in sigs.items():
            fn = getattr(self.lib, prefix + name, None)
            if fn is None:
                continue
            fn.restype = res
            fn.argtypes = args
            setattr(self, name, fn)

    def layout(self, D, G, bk, bv, body):
        lay = Layout()
        rc = self.layout_init(C.byref(lay), D, G, bk, bv, body)
        if rc != 0:
            raise ValueError("layout_init rc %d" % rc)
        return lay


_cache = {}


def oracle():
    if "oracle" not in _cache:
        _cache["oracle"] = Api(ORACLE_SO, "sjo_", _ORACLE_EXTRA)
    return _cache["oracle"]


def reference():
    """The reference compiled from /root/reference (None where it was not built)."""
    if "ref" not in _cache:
        _cache["ref"] = Api(REF_SO, "sj_kvarn_") if os.path.exists(REF_SO) else None
    return _cache["ref"]


def ptr(a, t=u8p):
    """numpy array -> ctypes pointer of type t"""
    return a.ctypes.data_as(t)
