"""ctypes binding of libmq.so (include/mq.h).  Device pointers are plain ints."""
import ctypes
import os

HERE = os.path.dirname(os.path.abspath(__file__))
# MQ_LIB_DIR selects another build of the same libraries (the host-sanitized one in _asan/)
LIB_DIR = os.environ.get("MQ_LIB_DIR") or HERE
LIB_PATH = os.path.join(LIB_DIR, "libmq.so")

TYPE_F32, TYPE_F16, TYPE_Q8_0, TYPE_Q4_K, TYPE_Q6_K, TYPE_Q8_K = 0, 1, 8, 12, 14, 15
Q8_0_X86, Q8_0_NEON, Q8_0_REF = 0, 1, 2
PATH_AUTO, PATH_GEMV, PATH_GEMM = 0, 1, 2
ATTN_KV_READY = 1
PRE_NONE, PRE_GELU_ERF, PRE_SILU_MUL = 0, 1, 2
TYPE_I32 = 26
BIN_ADD, BIN_SUB, BIN_MUL, BIN_DIV = 0, 1, 2, 3
UNARY_GELU_ERF, UNARY_GELU, UNARY_SILU, UNARY_RELU = 0, 1, 2, 3
NORM_LAYER, NORM_RMS = 0, 1
OP_GET_ROWS, OP_BINARY, OP_UNARY, OP_NORM, OP_CPY, OP_FLASH_ATTN, OP_ROPE = 0, 1, 2, 3, 4, 5, 6
ROPE_NORMAL, ROPE_NEOX = 0, 2
SORT_ASC, SORT_DESC = 0, 1

TYPE_NAMES = {TYPE_F32: "f32", TYPE_F16: "f16", TYPE_Q8_0: "q8_0", TYPE_Q4_K: "q4_K",
              TYPE_Q6_K: "q6_K", TYPE_Q8_K: "q8_K"}


class MQError(RuntimeError):
    pass


_lib = None

_c_i64 = ctypes.c_int64
_c_sz = ctypes.c_size_t
_c_vp = ctypes.c_void_p
_c_int = ctypes.c_int

# name -> (restype, argtypes)
_SIGS = {
    "mq_init": (_c_int, []),
    "mq_measure_mfma_i8": (_c_int, [_c_int, ctypes.POINTER(ctypes.c_double), ctypes.c_void_p]),
    "mq_last_error": (ctypes.c_char_p, []),
    "mq_gemv_max_m": (_c_int, []),
    "mq_q8_0_variant": (_c_int, []),
    "mq_set_q8_0_variant": (_c_int, [_c_int]),
    "mq_blck_size": (_c_i64, [_c_int]),
    "mq_type_size": (_c_sz, [_c_int]),
    "mq_row_size": (_c_sz, [_c_int, _c_i64]),
    "mq_vec_dot_type": (_c_int, [_c_int]),
    "mq_supports": (_c_int, [_c_int, _c_i64]),
    "mq_quantize_chunk": (_c_sz, [_c_int, _c_vp, _c_vp, _c_i64, _c_i64]),
    "mq_quantize_q8_0": (_c_int, [_c_vp, _c_i64, _c_vp, _c_i64, _c_i64, _c_int, _c_vp]),
    "mq_quantize_q8_K": (_c_int, [_c_vp, _c_i64, _c_vp, _c_i64, _c_i64, _c_vp]),
    "mq_quantize_f16": (_c_int, [_c_vp, _c_i64, _c_vp, _c_i64, _c_i64, _c_vp]),
    "mq_dequantize": (_c_int, [_c_int, _c_vp, _c_vp, _c_i64, _c_i64, _c_int, _c_vp]),
    "mq_gguf_bytes": (_c_sz, [_c_int, _c_i64, _c_i64]),
    "mq_gguf_bytes_aligned": (_c_sz, [_c_int, _c_i64, _c_i64]),
    "mq_weight_image_bytes": (_c_sz, [_c_int, _c_i64, _c_i64]),
    "mq_weight_prepare": (_c_int, [_c_int, _c_vp, _c_i64, _c_i64, _c_i64, _c_i64, _c_vp]),
    "mq_workspace_bytes": (_c_sz, [_c_int, _c_i64, _c_i64]),
    "mq_release_workspace": (_c_int, [_c_vp]),
    "mq_mul_mat": (_c_int, [_c_int, _c_vp, _c_i64, _c_i64, _c_vp, _c_i64, _c_i64, _c_vp, _c_i64, _c_vp,
                            _c_sz, _c_vp]),
    "mq_quantize_act": (_c_int, [_c_int, _c_vp, _c_i64, _c_i64, _c_i64, _c_vp, _c_sz, _c_int, _c_vp]),
    "mq_quantize_act_ex": (_c_int, [_c_int, _c_vp, _c_i64, _c_i64, _c_i64, _c_vp, _c_int, _c_vp, _c_sz, _c_int, _c_vp]),
    "mq_quantize_act_silu_mul": (_c_int, [_c_int, _c_vp, _c_vp, _c_i64, _c_i64, _c_i64, _c_vp, _c_sz, _c_int, _c_vp]),
    "mq_mul_mat_q": (_c_int, [_c_int, _c_vp, _c_i64, _c_i64, _c_vp, _c_i64, _c_vp, _c_i64, _c_int, _c_vp]),
    "mq_mul_mat_path": (_c_int, [_c_int, _c_i64, _c_i64, _c_i64]),
    "mq_mul_mat_q_ex": (_c_int, [_c_int, _c_vp, _c_i64, _c_i64, _c_vp, _c_i64, _c_vp, _c_i64, _c_vp, _c_int, _c_vp]),
    "mq_mul_mat_q_requant": (_c_int, [_c_int, _c_vp, _c_i64, _c_i64, _c_vp, _c_i64, _c_vp, _c_int, _c_int, _c_vp,
                                      _c_sz, _c_vp]),
    "mq_mul_mat_q_requant_supported": (_c_int, [_c_int, _c_int, _c_i64, _c_i64]),
    "mq_mul_mat_q_swiglu_supported": (_c_int, [_c_int, _c_i64, _c_i64]),
    "mq_mul_mat_q_swiglu": (_c_int, [_c_int, _c_vp, _c_i64, _c_i64, _c_vp, _c_i64, _c_vp, _c_i64, _c_vp]),
    "mq_mul_mat_q_qkv": (_c_int, [_c_int, ctypes.POINTER(_c_vp), ctypes.POINTER(_c_i64), _c_i64, _c_vp, _c_i64, _c_vp,
                                  _c_i64, ctypes.POINTER(_c_vp), _c_int, _c_int, _c_int, _c_vp, _c_sz, _c_vp]),
    "mq_mul_mat_q_group": (_c_int, [_c_int, _c_int, ctypes.POINTER(_c_vp), ctypes.POINTER(_c_i64), _c_i64, _c_vp,
                                    _c_i64, ctypes.POINTER(_c_vp), ctypes.POINTER(_c_i64), ctypes.POINTER(_c_vp),
                                    _c_int, _c_vp]),
    "mq_mul_mat_gemv": (_c_int, [_c_int, _c_int, ctypes.POINTER(_c_vp), ctypes.POINTER(_c_i64), _c_i64, _c_vp, _c_i64,
                                 _c_vp, _c_i64, _c_int, _c_i64, ctypes.POINTER(_c_vp), ctypes.POINTER(_c_i64),
                                 ctypes.POINTER(_c_vp), _c_vp]),
    "mq_mul_mat_ex": (_c_int, [_c_int, _c_vp, _c_i64, _c_i64, _c_vp, _c_i64, _c_i64, _c_vp, _c_i64, _c_vp,
                               _c_sz, _c_int, _c_vp]),
    "mq_mul_mat_noalloc": (_c_int, [_c_int, _c_vp, _c_i64, _c_i64, _c_vp, _c_i64, _c_i64, _c_vp, _c_i64, _c_int,
                                    _c_vp]),
    # include/mq_bert.h
    "mq_bert_create": (_c_vp, [_c_vp]),
    "mq_bert_free": (None, [_c_vp]),
    "mq_bert_set_embeddings": (_c_int, [_c_vp] * 6),
    "mq_bert_set_layer": (_c_int, [_c_vp, _c_int] + [_c_vp] * 16),
    "mq_bert_encode": (_c_int, [_c_vp, _c_vp, _c_vp, _c_int, _c_int, _c_vp, _c_vp, _c_vp]),
    # include/mq_gguf.h
    "mq_gguf_open": (_c_vp, [ctypes.c_char_p]),
    "mq_gguf_close": (None, [_c_vp]),
    "mq_gguf_version": (ctypes.c_uint32, [_c_vp]),
    "mq_gguf_alignment": (_c_sz, [_c_vp]),
    "mq_gguf_data_offset": (_c_sz, [_c_vp]),
    "mq_gguf_n_kv": (_c_i64, [_c_vp]),
    "mq_gguf_find_key": (_c_i64, [_c_vp, ctypes.c_char_p]),
    "mq_gguf_kv_key": (ctypes.c_char_p, [_c_vp, _c_i64]),
    "mq_gguf_kv_type": (_c_int, [_c_vp, _c_i64]),
    "mq_gguf_arr_type": (_c_int, [_c_vp, _c_i64]),
    "mq_gguf_arr_n": (_c_i64, [_c_vp, _c_i64]),
    "mq_gguf_arr_data": (_c_vp, [_c_vp, _c_i64]),
    "mq_gguf_arr_str": (ctypes.c_char_p, [_c_vp, _c_i64, _c_i64]),
    "mq_gguf_kv_data": (_c_vp, [_c_vp, _c_i64]),
    "mq_gguf_get_u32": (ctypes.c_uint32, [_c_vp, ctypes.c_char_p, ctypes.c_uint32]),
    "mq_gguf_get_i32": (ctypes.c_int32, [_c_vp, ctypes.c_char_p, ctypes.c_int32]),
    "mq_gguf_get_f32": (ctypes.c_float, [_c_vp, ctypes.c_char_p, ctypes.c_float]),
    "mq_gguf_get_bool": (_c_int, [_c_vp, ctypes.c_char_p, _c_int]),
    "mq_gguf_get_str": (ctypes.c_char_p, [_c_vp, ctypes.c_char_p, ctypes.c_char_p]),
    "mq_gguf_n_tensors": (_c_i64, [_c_vp]),
    "mq_gguf_find_tensor": (_c_i64, [_c_vp, ctypes.c_char_p]),
    "mq_gguf_tensor_name": (ctypes.c_char_p, [_c_vp, _c_i64]),
    "mq_gguf_tensor_info": (_c_int, [_c_vp, _c_i64, _c_vp, _c_vp, _c_vp, _c_vp, _c_vp]),
    "mq_gguf_tensor_data": (_c_vp, [_c_vp, _c_i64]),
    "mq_bert_load": (_c_vp, [ctypes.c_char_p]),
    "mq_decoder_load": (_c_vp, [ctypes.c_char_p]),
    "mq_bert_get_hparams": (_c_int, [_c_vp, _c_vp]),
    "mq_decoder_get_hparams": (_c_int, [_c_vp, _c_vp]),
    # include/mq_decoder.h
    "mq_decoder_create": (_c_vp, [_c_vp]),
    "mq_decoder_free": (None, [_c_vp]),
    "mq_decoder_set_embeddings": (_c_int, [_c_vp] * 3),
    "mq_decoder_set_layer": (_c_int, [_c_vp, _c_int] + [_c_vp] * 11),
    "mq_decoder_encode": (_c_int, [_c_vp, _c_vp, _c_int, _c_int, _c_vp, _c_vp, _c_vp]),
    "mq_decoder_set_observer": (_c_int, [_c_vp, _c_vp, _c_vp]),
    "mq_qk_norm_rope": (_c_int, [_c_vp, _c_i64, _c_vp, _c_vp, ctypes.c_float, _c_int, _c_int, _c_int, _c_int,
                                 ctypes.c_float, _c_i64, _c_vp]),
    "mq_attention_workspace_bytes": (ctypes.c_size_t, [_c_int, _c_int, _c_int, _c_int]),
    "mq_attention": (_c_int, [_c_vp, _c_i64, _c_vp, _c_i64, _c_int, _c_int, _c_int, _c_int, _c_int, ctypes.c_float,
                              _c_int, _c_vp, ctypes.c_size_t, _c_vp]),
    # mq_ops.h entries are added after View is defined
}


class View(ctypes.Structure):
    """mq_view (include/mq_ops.h): ggml metadata of a strided tensor (ne[0] fastest, nb in bytes)."""
    _fields_ = [("data", _c_vp), ("type", _c_int), ("ne", _c_i64 * 4), ("nb", _c_sz * 4)]


_TORCH_TYPES = {"torch.float32": TYPE_F32, "torch.float16": TYPE_F16, "torch.int32": TYPE_I32,
                "torch.uint8": None}


def view(t, type=None, ne=None, nb=None):
    """mq_view of a torch tensor: ggml order (ne[0] = the last torch dim).  For byte tensors
    holding quantized rows pass type and the ggml ne / nb explicitly."""
    v = View()
    v.data = t.data_ptr() if t is not None else None
    if ne is None:
        shape = list(t.shape)[::-1] + [1] * (4 - t.dim())
        strides = [s_ * t.element_size() for s_ in list(t.stride())[::-1]]
        strides += [strides[-1] * shape[len(strides) - 1] if strides else t.element_size()] * (4 - len(strides))
        ne, nb = shape, strides
        type = _TORCH_TYPES[str(t.dtype)] if type is None else type
    v.type = type
    for i in range(4):
        v.ne[i] = ne[i]
        v.nb[i] = nb[i]
    return v


_PV = ctypes.POINTER(View)
_SIGS.update({
    "mq_op_get_rows": (_c_int, [_PV, _PV, _PV, _c_vp]),
    "mq_op_binary": (_c_int, [_c_int, _PV, _PV, _PV, _c_vp]),
    "mq_op_unary": (_c_int, [_c_int, _PV, _PV, _c_vp]),
    "mq_op_norm": (_c_int, [_c_int, _PV, _PV, _PV, ctypes.c_float, _c_vp, _c_vp, _c_vp]),
    "mq_op_norm_q8_0": (_c_int, [_c_int, _PV, _PV, _PV, ctypes.c_float, _c_vp, _c_vp, _c_vp, _c_sz, _c_vp]),
    "mq_op_norm_q8_K": (_c_int, [_c_int, _PV, _PV, _PV, _PV, ctypes.c_float, _c_vp, _c_vp, _c_sz, _c_vp]),
    "mq_op_cpy": (_c_int, [_PV, _PV, _c_vp]),
    "mq_op_flash_attn_workspace_bytes": (_c_sz, [_PV]),
    "mq_op_flash_attn": (_c_int, [_PV, _PV, _PV, _PV, _PV, ctypes.c_float, _c_vp, _c_sz, _c_vp]),
    "mq_op_get_rows_sum": (_c_int, [_c_int, ctypes.POINTER(_PV), ctypes.POINTER(_PV), _PV, _c_vp]),
    "mq_op_flash_attn_ex": (_c_int, [_PV, _PV, _PV, _PV, _PV, ctypes.c_float, _c_vp, _c_sz, _c_vp, _c_sz, _c_int,
                                     _c_vp]),
    "mq_op_flash_attn_q8_0": (_c_int, [_PV, _PV, _PV, _PV, _PV, ctypes.c_float, _c_vp, _c_sz, _c_vp, _c_sz, _c_vp]),
    "mq_op_mask_blocks_bytes": (_c_sz, [_PV, _PV, _PV]),
    "mq_op_mask_blocks": (_c_int, [_PV, _PV, _PV, _c_vp, _c_sz, _c_vp]),
    "mq_op_mask_is_zero": (_c_int, [_PV, _PV, _PV, _c_vp, _c_sz, ctypes.POINTER(ctypes.c_int), _c_vp]),
    "mq_op_mask_segments_bytes": (_c_sz, [_PV, _PV, _PV]),
    "mq_op_mask_segments": (_c_int, [_PV, _PV, _PV, _c_vp, _c_sz, ctypes.POINTER(_c_i64), _c_vp]),
    "mq_op_flash_attn_blocks": (_c_int, [_PV, _PV, _PV, _PV, _PV, ctypes.c_float, _c_vp, _c_vp, ctypes.c_float,
                                         _c_vp, _c_vp, _c_i64, _c_vp, _c_sz, _c_vp, _c_sz, _c_int, _c_int, _c_vp]),
    "mq_op_supported": (_c_int, [_c_int, _c_int, _PV, _PV, _PV, _PV, _PV]),
    "mq_op_mul_mat_id_workspace_bytes": (_c_sz, [_c_int, _c_i64, _c_i64, _c_i64]),
    "mq_op_mul_mat_id": (_c_int, [_c_int, _c_vp, _c_sz, _c_int, _c_i64, _c_i64, _PV, _PV, _PV, _c_vp, _c_sz, _c_vp]),
    "mq_op_mul_mat_id_device_workspace_bytes": (_c_sz, [_c_int, _c_int, _c_i64, _c_i64, _c_i64]),
    "mq_op_mul_mat_id_device": (_c_int, [_c_int, _c_vp, _c_sz, _c_int, _c_i64, _c_i64, _PV, _PV, _PV, _c_vp, _c_sz,
                                         _c_vp]),
    "mq_op_soft_max": (_c_int, [_PV, _PV, _PV, ctypes.c_float, _c_vp]),
    "mq_op_argsort": (_c_int, [_PV, _PV, _c_int, _c_vp]),
    "mq_op_repeat": (_c_int, [_PV, _PV, _c_vp]),
    "mq_op_mul_mat_f32": (_c_int, [_PV, _PV, _PV, _c_vp]),
    "mq_op_rope": (_c_int, [_PV, _PV, _PV, _PV, _c_int, _c_int, _c_int] + [ctypes.c_float] * 6 + [_c_vp]),
    "mq_op_rope_cache": (_c_int, [_PV, _PV, _c_int, _c_int] + [ctypes.c_float] * 6 + [_c_vp, _c_vp]),
    "mq_op_flash_attn_qk_norm_rope": (_c_int, [_PV, _PV, _PV, _PV, _PV, ctypes.c_float, _c_vp, _c_vp, ctypes.c_float,
                                               _c_vp, _c_vp, _c_sz, _c_vp, _c_sz, _c_vp]),
    "mq_op_rms_norm_rope": (_c_int, [_PV, ctypes.c_float, _c_vp, _PV, _PV, _PV, _c_int, _c_int, _c_int] +
                            [ctypes.c_float] * 6 + [_c_vp]),
})


# mq_decoder_observer (include/mq_decoder.h)
DECODER_OBSERVER = ctypes.CFUNCTYPE(None, ctypes.c_char_p, _c_int, _c_vp, _c_i64, _c_i64, _c_vp, _c_sz, _c_vp)


class DecoderHparams(ctypes.Structure):
    """mq_decoder_hparams (include/mq_decoder.h)."""
    _fields_ = [("n_layer", _c_int), ("n_embd", _c_int), ("n_head", _c_int), ("n_kv_head", _c_int),
                ("head_dim", _c_int), ("n_ff", _c_int), ("n_vocab", _c_int), ("rms_norm_eps", ctypes.c_float),
                ("rope_theta", ctypes.c_float), ("causal", _c_int), ("pooling", _c_int), ("wtype", _c_int)]


class BertHparams(ctypes.Structure):
    """mq_bert_hparams (include/mq_bert.h)."""
    _fields_ = [("n_layer", _c_int), ("n_embd", _c_int), ("n_head", _c_int), ("n_ff", _c_int),
                ("n_vocab", _c_int), ("n_max_pos", _c_int), ("n_type", _c_int),
                ("layer_norm_eps", ctypes.c_float), ("wtype", _c_int)]


def lib():
    """Load libmq.so (raises if it was not built: there is no fallback)."""
    global _lib
    if _lib is None:
        # libmq.so and torch's bundled HIP runtime share the soname
        # libamdhip64.so.7: importing torch first makes libmq bind to that same
        # runtime, so torch's device pointers and streams are valid in libmq.
        try:
            import torch  # noqa: F401
        except ImportError:
            pass
        if not os.path.exists(LIB_PATH):
            raise MQError(f"{LIB_PATH} is missing; run `python -c 'import __graft_entry__ as g; g.build()'`")
        L = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in _SIGS.items():
            f = getattr(L, name)
            f.restype = res
            f.argtypes = args
        _lib = L
    return _lib


def check(rc):
    """Raise MQError with the library's message when rc != 0."""
    if rc != 0:
        msg = lib().mq_last_error()
        raise MQError(f"libmq error {rc}: {msg.decode() if msg else ''}")
    return rc
