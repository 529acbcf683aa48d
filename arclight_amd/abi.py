"""ctypes mirror of include/arclight_fattn.h (structures and constants only).

Loading no library, this module is shared by the product binding
(arclight_amd._lib) and by the CPU oracle's binding, which implement the same
operator interface: ArcLight's NNML_OP_FLASH_ATTN_EXT node with src tensors
q, k, v, mask, sinks and op_params {scale, max_bias, logit_softcap, prec}
(nnml/src/tensor.cpp:1292-1338, nnml/src/ops/ops.cpp:1432-1445).
"""
import ctypes

AL_TYPE_F32 = 0
AL_TYPE_F16 = 1
AL_TYPE_Q4_0 = 2     # include/arclight_matmul.h
AL_TYPE_I32 = 26
AL_TYPE_I64 = 27

AL_PREC_DEFAULT = 0
AL_PREC_F32 = 10

AL_OK = 0
AL_FATTN_HINT_TAG = 0x31484C41    # "ALH1": op_params i32[4] of an nnml node carrying length hints
AL_ERR_INVALID = -1
AL_ERR_UNSUPPORTED = -2
AL_ERR_HIP = -3
AL_ERR_WORKSPACE = -4

STATUS_NAMES = {
    AL_OK: "AL_OK",
    AL_ERR_INVALID: "AL_ERR_INVALID",
    AL_ERR_UNSUPPORTED: "AL_ERR_UNSUPPORTED",
    AL_ERR_HIP: "AL_ERR_HIP",
    AL_ERR_WORKSPACE: "AL_ERR_WORKSPACE",
}

TYPE_SIZES = {AL_TYPE_F32: 4, AL_TYPE_F16: 2, AL_TYPE_I32: 4, AL_TYPE_I64: 8}

# Q4_0 blocks (nnml/include/nnml.h:646-650): 32 weights as an f16 scale and
# 16 bytes of nibbles, low nibbles the first 16 weights (types.cpp:337-350).
QK4_0 = 32
Q4_0_BLOCK_BYTES = 18


class AlTensor(ctypes.Structure):
    _fields_ = [
        ("data", ctypes.c_void_p),
        ("type", ctypes.c_int32),
        ("reserved", ctypes.c_int32),
        ("ne", ctypes.c_int64 * 4),
        ("nb", ctypes.c_uint64 * 4),
    ]


class AlFattnArgs(ctypes.Structure):
    _fields_ = [
        ("q", AlTensor),
        ("k", AlTensor),
        ("v", AlTensor),
        ("mask", AlTensor),
        ("sinks", AlTensor),
        ("dst", AlTensor),
        ("scale", ctypes.c_float),
        ("max_bias", ctypes.c_float),
        ("logit_softcap", ctypes.c_float),
        ("prec", ctypes.c_int32),
        ("kv_len", ctypes.c_int64),
        ("causal_pos0", ctypes.c_int64),
        ("stream", ctypes.c_void_p),
        ("workspace", ctypes.c_void_p),
        ("workspace_bytes", ctypes.c_uint64),
        ("dyn_len", ctypes.c_void_p),
    ]


def make_tensor(data, typ, ne, nb=None):
    """Builds an AlTensor. `ne` is nnml order (ne[0] fastest); `nb` defaults to
    contiguous byte strides."""
    t = AlTensor()
    t.data = data if data else None
    t.type = typ
    ne = list(ne) + [1] * (4 - len(ne))
    if nb is None:
        nb = [TYPE_SIZES[typ]]
        for i in range(1, 4):
            nb.append(nb[i - 1] * ne[i - 1])
    for i in range(4):
        t.ne[i] = int(ne[i])
        t.nb[i] = int(nb[i])
    return t


def empty_tensor():
    return make_tensor(None, AL_TYPE_F32, [0, 0, 0, 0], [0, 0, 0, 0])


# Physical numpy layouts of each operand, as the axis of the numpy array that
# holds nnml dim ne0..ne3. These are the layouts the Qwen3 graph produces
# (nnml/src/cgraph.cpp:250-258, 1072-1102; store at arm.cpp:2431):
#   q     array (B, T, Hq, D)        f32  -> ne = [D, T, Hq, B]
#   k, v  array (B, n_kv, Hkv, D)    f16  -> ne = [D, n_kv, Hkv, B]
#   mask  array (m3, m2, rows, n_kv) f16  -> ne = [n_kv, rows, m2, m3]
#   dst   array (B, T, Hq, D)        f32  -> ne = [D, Hq, T, B]
Q_AXES = (3, 1, 2, 0)
KV_AXES = (3, 1, 2, 0)
MASK_AXES = (3, 2, 1, 0)
DST_AXES = (3, 2, 1, 0)


def tensor_desc(data, typ, shape, strides, axes):
    """AlTensor for an array of numpy `shape`/`strides` (bytes) whose nnml dim
    i lives on numpy axis axes[i]."""
    ne = [int(shape[a]) for a in axes]
    nb = [int(strides[a]) for a in axes]
    return make_tensor(data, typ, ne, nb)


# include/arclight_kv.h
class AlUbatch(ctypes.Structure):
    _fields_ = [
        ("n_tokens", ctypes.c_int32),
        ("pos", ctypes.POINTER(ctypes.c_int32)),
        ("seq_mask", ctypes.POINTER(ctypes.c_uint64)),
    ]


class AlKvRingParams(ctypes.Structure):
    _fields_ = [
        ("n_layer", ctypes.c_uint32),
        ("kv_size", ctypes.c_uint32),
        ("n_seq_max", ctypes.c_uint32),
        ("n_pad", ctypes.c_uint32),
        ("n_head_kv", ctypes.c_uint32),
        ("head_dim", ctypes.c_uint32),
        ("unified", ctypes.c_int32),
    ]


# include/arclight_prologue.h
AL_ROPE_NORMAL = 0
AL_ROPE_NEOX = 2


class AlRopeParams(ctypes.Structure):
    _fields_ = [
        ("n_dims", ctypes.c_int32),
        ("mode", ctypes.c_int32),
        ("n_ctx_orig", ctypes.c_int32),
        ("freq_base", ctypes.c_float),
        ("freq_scale", ctypes.c_float),
        ("ext_factor", ctypes.c_float),
        ("attn_factor", ctypes.c_float),
        ("beta_fast", ctypes.c_float),
        ("beta_slow", ctypes.c_float),
    ]


class AlAttnInputsArgs(ctypes.Structure):
    """al_attn_inputs_args (include/arclight_prologue.h)."""
    _fields_ = [
        ("q", AlTensor), ("q_w", AlTensor), ("k", AlTensor), ("k_w", AlTensor), ("v", AlTensor),
        ("pos", AlTensor), ("rows", AlTensor), ("q_out", AlTensor), ("k_cache", AlTensor), ("v_cache", AlTensor),
        ("eps", ctypes.c_float),
        ("rope", ctypes.POINTER(AlRopeParams)),
    ]


def qwen3_rope(n_ctx_orig=40960):
    """Qwen3's rope_ext parameters (models/qwen3.cpp:49-55)."""
    return AlRopeParams(128, AL_ROPE_NEOX, n_ctx_orig, 1000000.0, 1.0, 0.0, 1.0, 32.0, 1.0)
