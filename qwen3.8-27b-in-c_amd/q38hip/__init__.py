"""Python host binding of libq38hip (the gfx950 decode hot path).

Thin ctypes layer over the C ABI in include/q38hip.h.  Device memory and
streams come from PyTorch (ROCm build); every computation runs in the HIP
kernels of libq38hip.so.  There is no CPU fallback: importing this module
without the built library raises.

Names mirror the reference kernel ABI (include/qwen38/qwen38_quant.h of
shyringo/qwen3.8-27b-in-c): quantize_q8_k, tensor_gemv_q8_k,
tensor_gemm_q8_k, plus device-resident forms that take torch tensors.
"""
import ctypes
import os

import numpy as np

PACKAGE_DIR = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB_PATH = os.path.join(PACKAGE_DIR, "libq38hip.so")

Q4_K, Q6_K, IQ1_M = 12, 14, 29
BLOCK_BYTES = {Q4_K: 144, Q6_K: 210, IQ1_M: 56}
Q8K_BYTES = 292
Q8K_DTYPE = np.dtype([("scale", "<f4"), ("quants", "i1", (256,)), ("sums", "<i2", (16,))])


class GGUFString(ctypes.Structure):
    _fields_ = [("data", ctypes.c_char_p), ("length", ctypes.c_uint64)]


class GGUFTensor(ctypes.Structure):
    """Q38GGUFTensor: shape[0] = input width, shape[1] = rows."""
    _fields_ = [("name", GGUFString), ("n_dims", ctypes.c_uint32),
                ("shape", ctypes.c_uint64 * 8), ("type", ctypes.c_uint32),
                ("offset", ctypes.c_uint64), ("nbytes", ctypes.c_uint64),
                ("data", ctypes.c_void_p), ("iq1_s_repack", ctypes.c_void_p)]


def make_tensor(data_ptr, qtype, width, rows, nbytes=0):
    tensor = GGUFTensor()
    tensor.n_dims = 2
    tensor.shape[0] = width
    tensor.shape[1] = rows
    tensor.type = qtype
    tensor.nbytes = nbytes
    tensor.data = data_ptr
    return tensor


# Every symbol the C header declares (tests check the library exports them).
EXPORTS = ("q38_f16_to_f32", "q38_quantize_q8_k", "q38_tensor_gemv_q8_k", "q38_tensor_gemm_q8_k",
           "q38_tensor_row_f32", "q38_tensor_dot_row_f32", "q38_tensor_gemv_f32", "q38_tensor_gemm_f32",
           "q38_prepare_iq1_s_repacks", "q38_release_iq1_s_repacks", "q38hip_gemm_f32", "q38hip_row_f32",
           "q38hip_quantize_q8_k", "q38hip_gemm_q8_k", "q38hip_argmax", "q38hip_argmax_noalloc", "q38hip_accept",
           "q38hip_tiled_q4k_bytes", "q38hip_repack_q4k_tiles", "q38hip_gemm_q8_k_tiled", "q38hip_attention_rows",
           "q38hip_tiled_iq1m_bytes", "q38hip_repack_iq1m_tiles", "q38hip_gemm_q8_k_iq1m_tiled",
           "q38hip_sample", "q38hip_last_error", "q38hip_synchronize",
           "q38_model_open_gguf", "q38_model_attach_mtp_gguf", "q38_model_close", "q38_model_reset",
           "q38_model_forward_token", "q38_model_prefill", "q38_model_enable_mtp", "q38_model_mtp_forward",
           "q38_model_speculative_greedy", "q38_model_forward_token_layers", "q38_model_vocab_size",
           "q38_model_position", "q38_model_context_length", "q38hip_model_sample",
           "q38hip_model_forward_sample")


def load_library(path=LIB_PATH):
    if not os.path.exists(path):
        raise RuntimeError("libq38hip.so is not built (run __graft_entry__.build() or "
                           "make -C qwen3.8-27b-in-c_amd)")
    lib = ctypes.CDLL(path)
    vp, u32, u64 = ctypes.c_void_p, ctypes.c_uint32, ctypes.c_uint64
    lib.q38_f16_to_f32.restype = ctypes.c_float
    lib.q38_f16_to_f32.argtypes = [ctypes.c_uint16]
    lib.q38_quantize_q8_k.argtypes = [vp, vp, u64]
    lib.q38_tensor_gemv_q8_k.argtypes = [vp, vp, u64, ctypes.POINTER(GGUFTensor)]
    lib.q38_tensor_gemm_q8_k.argtypes = [vp, vp, u32, u64, ctypes.POINTER(GGUFTensor)]
    lib.q38hip_quantize_q8_k.argtypes = [vp, vp, u64, u32, vp]
    lib.q38_tensor_row_f32.argtypes = [vp, ctypes.POINTER(GGUFTensor), u64]
    lib.q38_tensor_dot_row_f32.argtypes = [vp, vp, ctypes.POINTER(GGUFTensor), u64]
    lib.q38_tensor_gemv_f32.argtypes = [vp, vp, ctypes.POINTER(GGUFTensor)]
    lib.q38_tensor_gemm_f32.argtypes = [vp, vp, u32, u64, ctypes.POINTER(GGUFTensor)]
    lib.q38_prepare_iq1_s_repacks.argtypes = [vp]
    lib.q38_release_iq1_s_repacks.restype = None
    lib.q38_release_iq1_s_repacks.argtypes = [vp]
    lib.q38hip_gemm_f32.argtypes = [vp, vp, u32, u64, ctypes.POINTER(GGUFTensor), vp]
    lib.q38hip_row_f32.argtypes = [vp, ctypes.POINTER(GGUFTensor), u64, u32, vp]
    lib.q38hip_gemm_q8_k.argtypes = [vp, vp, u32, u64, ctypes.POINTER(GGUFTensor), vp]
    lib.q38hip_tiled_q4k_bytes.restype = u64
    lib.q38hip_tiled_q4k_bytes.argtypes = [u32, u64]
    lib.q38hip_repack_q4k_tiles.argtypes = [vp, vp, u32, u64, vp]
    lib.q38hip_gemm_q8_k_tiled.argtypes = [vp, vp, u32, u64, vp, u32, vp]
    lib.q38hip_tiled_iq1m_bytes.restype = u64
    lib.q38hip_tiled_iq1m_bytes.argtypes = [u32, u64]
    lib.q38hip_repack_iq1m_tiles.argtypes = [vp, vp, u32, u64, vp]
    lib.q38hip_gemm_q8_k_iq1m_tiled.argtypes = [vp, vp, u32, u64, vp, u32, vp]
    lib.q38hip_argmax.argtypes = [vp, vp, u32, u32, vp]
    lib.q38hip_argmax_noalloc.argtypes = [vp, vp, u32, u32, vp]
    lib.q38hip_accept.argtypes = [vp, vp, vp, u32, vp]
    lib.q38hip_attention_rows.argtypes = [vp, vp, vp, vp, vp, u64, vp, vp, vp, vp, u32, u32, u32, vp]
    lib.q38hip_sample.argtypes = [vp, ctypes.POINTER(ctypes.c_uint64), vp, u32, ctypes.c_float, ctypes.c_float,
                                  ctypes.c_float, u32, vp, u32, vp]
    lib.q38hip_last_error.restype = ctypes.c_char_p
    lib.q38hip_last_error.argtypes = []
    lib.q38hip_synchronize.argtypes = []
    return lib


_LIB = None


def lib():
    global _LIB
    if _LIB is None:
        _LIB = load_library()
    return _LIB


def last_error():
    return lib().q38hip_last_error().decode()


def _check(ok, what):
    if not ok:
        raise RuntimeError("%s failed: %s" % (what, last_error()))


def _stream():
    import torch
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


def _dev_ptr(tensor):
    if not tensor.is_cuda:
        raise ValueError("expected a device tensor")
    if not tensor.is_contiguous():
        raise ValueError("expected a contiguous tensor")
    return ctypes.c_void_p(tensor.data_ptr())


# ---- sampler state (host side of include/qwen38/qwen38_sampler.h) ----------

class Sampler:
    """The Q38Sampler fields (include/qwen38/qwen38_sampler.h:10-18) with
    q38_sampler_init's defaults (src/qwen38/qwen38_sampler.c:22-32) and
    q38_sampler_observe (:34-38).  `presence` is a numpy uint8 array or None;
    `state` advances with every sampling call made through it."""

    GOLDEN = 0x9E3779B97F4A7C15

    def __init__(self, seed=0, temperature=1.0, top_p=0.95, presence_penalty=0.0, top_k=20, presence=None):
        self.state = int(seed) if seed else self.GOLDEN
        self.temperature = float(temperature)
        self.top_p = float(top_p)
        self.presence_penalty = float(presence_penalty)
        self.top_k = int(top_k)
        self.presence = presence

    def observe(self, token):
        if self.presence is not None and 0 <= token < self.presence.size:
            self.presence[token] = 1


# ---- device-resident API (torch tensors on the GPU) --------------------------

def quantize_q8_k(x):
    """x: float32 [rows, length] (or [length]) on the GPU -> uint8 Q8_K blocks."""
    import torch
    if x.dtype != torch.float32:
        raise ValueError("expected float32 input")
    rows = x.shape[0] if x.dim() == 2 else 1
    length = x.shape[-1]
    out = torch.empty(rows * (length // 256) * Q8K_BYTES, dtype=torch.uint8, device=x.device)
    _check(lib().q38hip_quantize_q8_k(_dev_ptr(out), _dev_ptr(x), length, rows, _stream()),
           "q38hip_quantize_q8_k")
    return out


def gemm_q8_k(weights, qtype, width, rows, xq, batch, out=None):
    """weights: uint8 GGUF rows on the GPU; xq: batch * width/256 Q8_K blocks.
    Returns float32 [batch, rows] (batch-major, as the reference GEMM)."""
    import torch
    if out is None:
        out = torch.empty((batch, rows), dtype=torch.float32, device=weights.device)
    tensor = make_tensor(weights.data_ptr(), qtype, width, rows, weights.numel())
    _check(lib().q38hip_gemm_q8_k(_dev_ptr(out), _dev_ptr(xq), batch, width, ctypes.byref(tensor),
                                  _stream()), "q38hip_gemm_q8_k")
    return out


def gemm_f32(weights, qtype, width, rows, x, out=None):
    """weights: uint8 GGUF rows on the GPU; x: float32 [batch, width] on the
    GPU.  Returns float32 [batch, rows] (q38_tensor_gemm_f32)."""
    import torch
    x2 = x if x.dim() == 2 else x.reshape(1, -1)
    if out is None:
        out = torch.empty((x2.shape[0], rows), dtype=torch.float32, device=weights.device)
    tensor = make_tensor(weights.data_ptr(), qtype, width, rows, weights.numel())
    _check(lib().q38hip_gemm_f32(_dev_ptr(out), _dev_ptr(x2), x2.shape[0], width, ctypes.byref(tensor), _stream()),
           "q38hip_gemm_f32")
    return out


def row_f32(weights, qtype, width, rows, first, count=1):
    """Rows first .. first + count - 1 of a GGUF matrix on the GPU as
    float32 [count, width] (q38_tensor_row_f32)."""
    import torch
    out = torch.empty((count, width), dtype=torch.float32, device=weights.device)
    tensor = make_tensor(weights.data_ptr(), qtype, width, rows, weights.numel())
    _check(lib().q38hip_row_f32(_dev_ptr(out), ctypes.byref(tensor), first, count, _stream()), "q38hip_row_f32")
    return out


def repack_q4k_tiles(weights, width, rows):
    """weights: uint8 row-major Q4_K rows on the GPU -> uint8 tiled copy."""
    import torch
    nbytes = int(lib().q38hip_tiled_q4k_bytes(rows, width))
    if nbytes == 0:
        raise ValueError("bad tiled shape")
    out = torch.empty(nbytes, dtype=torch.uint8, device=weights.device)
    _check(lib().q38hip_repack_q4k_tiles(_dev_ptr(out), _dev_ptr(weights), rows, width, _stream()),
           "q38hip_repack_q4k_tiles")
    return out


def gemm_q8_k_tiled(tiled, width, rows, xq, batch, out=None):
    """tiled: uint8 tiled Q4_K copy on the GPU; returns float32 [batch, rows]."""
    import torch
    if out is None:
        out = torch.empty((batch, rows), dtype=torch.float32, device=tiled.device)
    _check(lib().q38hip_gemm_q8_k_tiled(_dev_ptr(out), _dev_ptr(xq), batch, width, _dev_ptr(tiled), rows,
                                        _stream()), "q38hip_gemm_q8_k_tiled")
    return out


def repack_iq1m_tiles(weights, width, rows):
    """weights: uint8 row-major IQ1_M rows on the GPU -> uint8 tiled copy."""
    import torch
    nbytes = int(lib().q38hip_tiled_iq1m_bytes(rows, width))
    if nbytes == 0:
        raise ValueError("bad tiled shape")
    out = torch.empty(nbytes, dtype=torch.uint8, device=weights.device)
    _check(lib().q38hip_repack_iq1m_tiles(_dev_ptr(out), _dev_ptr(weights), rows, width, _stream()),
           "q38hip_repack_iq1m_tiles")
    return out


def gemm_q8_k_iq1m_tiled(tiled, width, rows, xq, batch, out=None):
    """tiled: uint8 tiled IQ1_M copy on the GPU; returns float32 [batch, rows]."""
    import torch
    if out is None:
        out = torch.empty((batch, rows), dtype=torch.float32, device=tiled.device)
    _check(lib().q38hip_gemm_q8_k_iq1m_tiled(_dev_ptr(out), _dev_ptr(xq), batch, width, _dev_ptr(tiled), rows,
                                             _stream()), "q38hip_gemm_q8_k_iq1m_tiled")
    return out


def argmax(values):
    """values: float32 [rows, count] on the GPU -> int32 [rows] first-max indices."""
    import torch
    values2 = values if values.dim() == 2 else values.reshape(1, -1)
    out = torch.empty(values2.shape[0], dtype=torch.int32, device=values.device)
    _check(lib().q38hip_argmax(_dev_ptr(out), _dev_ptr(values2), values2.shape[1], values2.shape[0],
                               _stream()), "q38hip_argmax")
    return out


def argmax_noalloc(values, out=None):
    """q38hip_argmax_noalloc: as argmax(), with the partial maxima in the
    library's fixed device array (no allocation by the library)."""
    import torch
    values2 = values if values.dim() == 2 else values.reshape(1, -1)
    if out is None:
        out = torch.empty(values2.shape[0], dtype=torch.int32, device=values.device)
    _check(lib().q38hip_argmax_noalloc(_dev_ptr(out), _dev_ptr(values2), values2.shape[1], values2.shape[0],
                                       _stream()), "q38hip_argmax_noalloc")
    return out


def sample(logits, sampler, presence=None, out=None):
    """q38hip_sample: one token from float32 logits [vocabulary] on the GPU,
    drawn as q38_sample draws it; `sampler` (a Sampler) supplies the
    parameters and its state advances.  presence: a uint8 device tensor or
    None (then sampler.presence is not used).  Returns an int32 [1] device
    tensor."""
    import torch
    if logits.dtype != torch.float32:
        raise ValueError("expected float32 logits")
    if out is None:
        out = torch.empty(1, dtype=torch.int32, device=logits.device)
    state = ctypes.c_uint64(sampler.state)
    _check(lib().q38hip_sample(_dev_ptr(out), ctypes.byref(state), _dev_ptr(logits), logits.numel(),
                               sampler.temperature, sampler.top_p, sampler.presence_penalty, sampler.top_k,
                               None if presence is None else _dev_ptr(presence),
                               0 if presence is None else presence.numel(), _stream()), "q38hip_sample")
    sampler.state = state.value
    return out


def accept(targets, drafts):
    """targets, drafts: int32 [rows] on the GPU -> int32 [rows + 3] result words."""
    import torch
    rows = targets.numel()
    out = torch.zeros(rows + 3, dtype=torch.int32, device=targets.device)
    _check(lib().q38hip_accept(_dev_ptr(out), _dev_ptr(targets), _dev_ptr(drafts), rows, _stream()),
           "q38hip_accept")
    return out


def value_pitch(context):
    """positions per channel row of the channel-major value cache"""
    return (int(context) + 31) // 32 * 32


def attention_rows(rows_in, q_norm, k_norm, key_cache, value_cache, position):
    """Full-attention core over the rows of rows_in (float32 [rows, 14336] on
    the GPU: 24 heads x (256 q | 256 gate), then key [1024], then value
    [1024]) at positions position + t; key_cache: float32 [context, 1024],
    value_cache: channel-major float32 [1024, value_pitch(context)], both on
    the GPU and updated in place.  Returns (attention float32 [rows, 6144],
    its Q8_K blocks uint8 [rows * 24 * 292])."""
    import torch
    rows, stride = rows_in.shape
    context = key_cache.shape[0]
    if tuple(value_cache.shape) != (1024, value_pitch(context)):
        raise ValueError("value_cache must be [1024, value_pitch(context)]")
    out = torch.empty((rows, 6144), dtype=torch.float32, device=rows_in.device)
    q8k = torch.empty(rows * 24 * Q8K_BYTES, dtype=torch.uint8, device=rows_in.device)
    base = rows_in.data_ptr()
    _check(lib().q38hip_attention_rows(_dev_ptr(out), _dev_ptr(q8k), _dev_ptr(rows_in),
                                       ctypes.c_void_p(base + 12288 * 4), ctypes.c_void_p(base + 13312 * 4), stride,
                                       _dev_ptr(q_norm), _dev_ptr(k_norm), _dev_ptr(key_cache),
                                       _dev_ptr(value_cache), context, position, rows, _stream()),
           "q38hip_attention_rows")
    return out, q8k


# ---- host-pointer drop-ins (numpy arrays) ------------------------------------

def host_quantize_q8_k(x):
    x = np.ascontiguousarray(x, dtype=np.float32).reshape(-1)
    out = np.zeros(x.size // 256, dtype=Q8K_DTYPE)
    _check(lib().q38_quantize_q8_k(out.ctypes.data, x.ctypes.data, x.size), "q38_quantize_q8_k")
    return out


def host_tensor_gemm_q8_k(qtype, data, rows, q8k, batch):
    width = q8k.size // batch * 256
    tensor = make_tensor(data.ctypes.data, qtype, width, rows, data.nbytes)
    out = np.zeros(batch * rows, dtype=np.float32)
    _check(lib().q38_tensor_gemm_q8_k(out.ctypes.data, q8k.ctypes.data, batch, width, ctypes.byref(tensor)),
           "q38_tensor_gemm_q8_k")
    return out.reshape(batch, rows)


def host_tensor_gemv_q8_k(qtype, data, rows, q8k):
    width = q8k.size * 256
    tensor = make_tensor(data.ctypes.data, qtype, width, rows, data.nbytes)
    out = np.zeros(rows, dtype=np.float32)
    _check(lib().q38_tensor_gemv_q8_k(out.ctypes.data, q8k.ctypes.data, width, ctypes.byref(tensor)),
           "q38_tensor_gemv_q8_k")
    return out
