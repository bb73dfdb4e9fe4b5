"""ctypes front end for the CPU checkers -- TEST INFRASTRUCTURE ONLY.

* ``Oracle``  wraps oracle/liboracle.so, our C restatement of the reference
  kernels (q38_oracle.c, each function citing the reference lines it follows).
* ``Reference`` wraps oracle/_ref/libq38ref.so, the reference's own C sources
  compiled where they lie (oracle/Makefile), when that library was built.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg import
this module.  The product library never does.
"""
import ctypes
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ORACLE_SO = os.path.join(HERE, "liboracle.so")
REF_SO = os.path.join(HERE, "_ref", "libq38ref.so")

Q4_K, Q6_K, IQ1_M = 12, 14, 29
BLOCK_BYTES = {Q4_K: 144, Q6_K: 210, IQ1_M: 56}

# Every matrix format the reference model accepts (src/qwen38/qwen38_model.c:
# 172-189): GGML type id -> (elements per block, bytes per block).
F32, F16, Q8_0, Q2_K, Q3_K, Q5_K, IQ2_XXS, IQ2_XS, IQ3_XXS, IQ1_S, IQ4_NL, IQ3_S, IQ2_S, IQ4_XS, BF16 = (
    0, 1, 8, 10, 11, 13, 16, 17, 18, 19, 20, 21, 22, 23, 30)
FORMATS = {F32: (1, 4), F16: (1, 2), BF16: (1, 2), Q8_0: (32, 34), Q2_K: (256, 84), Q3_K: (256, 110),
           Q4_K: (256, 144), Q5_K: (256, 176), Q6_K: (256, 210), IQ2_XXS: (256, 66), IQ2_XS: (256, 74),
           IQ2_S: (256, 82), IQ3_XXS: (256, 98), IQ3_S: (256, 110), IQ4_XS: (256, 136), IQ4_NL: (32, 18),
           IQ1_S: (256, 50), IQ1_M: (256, 56)}
FORMAT_NAMES = {F32: "F32", F16: "F16", BF16: "BF16", Q8_0: "Q8_0", Q2_K: "Q2_K", Q3_K: "Q3_K", Q4_K: "Q4_K",
                Q5_K: "Q5_K", Q6_K: "Q6_K", IQ2_XXS: "IQ2_XXS", IQ2_XS: "IQ2_XS", IQ2_S: "IQ2_S",
                IQ3_XXS: "IQ3_XXS", IQ3_S: "IQ3_S", IQ4_XS: "IQ4_XS", IQ4_NL: "IQ4_NL", IQ1_S: "IQ1_S",
                IQ1_M: "IQ1_M"}
# formats whose GEMV takes Q8_K activations (q38_matrix_type_q8_k, :172-182);
# the rest take fp32 activations through q38_tensor_gemv_f32
Q8K_FORMATS = (Q2_K, Q3_K, Q4_K, Q5_K, Q6_K, IQ2_XXS, IQ2_XS, IQ3_XXS, IQ4_NL, IQ3_S, IQ2_S, IQ4_XS, IQ1_S, IQ1_M)
F32_FORMATS = (F32, F16, BF16, Q8_0)


def row_bytes(qtype, width):
    elements, nbytes = FORMATS[qtype]
    return width // elements * nbytes

# Q38Q8KBlock (include/qwen38/qwen38_quant.h:14-18): 292 bytes, no padding.
Q8K_DTYPE = np.dtype([("scale", "<f4"), ("quants", "i1", (256,)), ("sums", "<i2", (16,))])
assert Q8K_DTYPE.itemsize == 292

_f32p = ctypes.POINTER(ctypes.c_float)
_u32p = ctypes.POINTER(ctypes.c_uint32)


def _ptr(array):
    return ctypes.c_void_p(array.ctypes.data)


class Q38Sampler(ctypes.Structure):
    """include/qwen38/qwen38_sampler.h:10-18"""
    _fields_ = [("state", ctypes.c_uint64), ("temperature", ctypes.c_float), ("top_p", ctypes.c_float),
                ("presence_penalty", ctypes.c_float), ("top_k", ctypes.c_uint32),
                ("presence", ctypes.c_void_p), ("presence_size", ctypes.c_uint32)]


def _sample_args(logits, presence):
    logits = np.ascontiguousarray(logits, dtype=np.float32)
    if presence is not None:
        presence = np.ascontiguousarray(presence, dtype=np.uint8)
    return logits, presence


class GGUFString(ctypes.Structure):
    _fields_ = [("data", ctypes.c_char_p), ("length", ctypes.c_uint64)]


class GGUFTensor(ctypes.Structure):
    """Q38GGUFTensor (include/qwen38/qwen38_gguf.h:68-77)."""
    _fields_ = [("name", GGUFString), ("n_dims", ctypes.c_uint32),
                ("shape", ctypes.c_uint64 * 8), ("type", ctypes.c_uint32),
                ("offset", ctypes.c_uint64), ("nbytes", ctypes.c_uint64),
                ("data", ctypes.c_void_p), ("iq1_s_repack", ctypes.c_void_p)]


def make_tensor(data, qtype, width, rows):
    tensor = GGUFTensor()
    tensor.n_dims = 2
    tensor.shape[0] = width
    tensor.shape[1] = rows
    tensor.type = qtype
    tensor.nbytes = data.nbytes
    tensor.data = data.ctypes.data
    return tensor


class Oracle:
    def __init__(self, path=ORACLE_SO):
        if not os.path.exists(path):
            raise RuntimeError("oracle library missing: run make -C oracle")
        lib = ctypes.CDLL(path)
        lib.orc_f16_to_f32.restype = ctypes.c_float
        lib.orc_f16_to_f32.argtypes = [ctypes.c_uint16]
        lib.orc_nearest_int.restype = ctypes.c_int
        lib.orc_nearest_int.argtypes = [ctypes.c_float]
        lib.orc_quantize_q8_k.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_uint64]
        lib.orc_block_ints.argtypes = [ctypes.c_uint32, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p]
        lib.orc_gemv_q8_k.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_uint64,
                                      ctypes.c_uint32, ctypes.c_void_p, ctypes.c_uint64]
        lib.orc_gemm_q8_k.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_uint32, ctypes.c_uint64,
                                      ctypes.c_uint32, ctypes.c_void_p, ctypes.c_uint64]
        lib.orc_row_f32.argtypes = [ctypes.c_void_p, ctypes.c_uint32, ctypes.c_void_p,
                                    ctypes.c_uint64, ctypes.c_uint64]
        lib.orc_argmax.restype = ctypes.c_uint32
        lib.orc_argmax.argtypes = [ctypes.c_void_p, ctypes.c_uint32]
        lib.orc_accept.restype = ctypes.c_uint32
        lib.orc_accept.argtypes = [ctypes.c_void_p, ctypes.c_uint32, ctypes.c_uint32, ctypes.c_void_p,
                                   _u32p, _u32p, ctypes.c_void_p]
        lib.orc_iq1m_grid_entry.argtypes = [ctypes.c_uint32, ctypes.c_void_p]
        lib.orc_attention_decode.argtypes = [ctypes.c_void_p] * 8 + [ctypes.c_uint32]
        vp, u32, u64 = ctypes.c_void_p, ctypes.c_uint32, ctypes.c_uint64
        lib.orc_format_gemv_q8_k.argtypes = [vp, vp, u64, u32, vp, u64]
        lib.orc_format_gemv_f32.argtypes = [vp, vp, u64, u32, vp, u64]
        lib.orc_format_row_f32.argtypes = [vp, u32, vp, u64, u64]
        lib.orc_format_block_lanes.argtypes = [u32, vp, vp, vp, ctypes.POINTER(ctypes.c_int32)]
        lib.orc_format_block_decode.argtypes = [u32, vp, vp, vp]
        lib.orc_sample.argtypes = [ctypes.c_void_p, ctypes.POINTER(ctypes.c_uint64), ctypes.c_void_p,
                                   ctypes.c_uint32, ctypes.c_float, ctypes.c_float, ctypes.c_float,
                                   ctypes.c_uint32, ctypes.c_void_p, ctypes.c_uint32]
        self.lib = lib

    def f16_to_f32(self, bits):
        return self.lib.orc_f16_to_f32(int(bits))

    def quantize(self, x):
        x = np.ascontiguousarray(x, dtype=np.float32)
        out = np.zeros(x.size // 256, dtype=Q8K_DTYPE)
        if not self.lib.orc_quantize_q8_k(_ptr(out), _ptr(x), x.size):
            raise ValueError("length must be a multiple of 256")
        return out

    def block_ints(self, qtype, block, q8k_block):
        ints = np.zeros(12, dtype=np.int32)
        n = self.lib.orc_block_ints(qtype, _ptr(block), _ptr(q8k_block), _ptr(ints))
        return ints[:n]

    def gemv(self, qtype, data, rows, q8k):
        out = np.zeros(rows, dtype=np.float32)
        if not self.lib.orc_format_gemv_q8_k(_ptr(out), _ptr(q8k), q8k.size * 256, qtype, _ptr(data), rows):
            raise ValueError("bad GEMV arguments")
        return out

    def gemv_f32(self, qtype, data, rows, x):
        """q38_tensor_gemv_f32 restated: fp32 input x [width]."""
        x = np.ascontiguousarray(x, dtype=np.float32)
        out = np.zeros(rows, dtype=np.float32)
        if not self.lib.orc_format_gemv_f32(_ptr(out), _ptr(x), x.size, qtype, _ptr(data), rows):
            raise ValueError("bad float GEMV arguments")
        return out

    def format_row_f32(self, qtype, data, width, row):
        """q38_tensor_row_f32 restated, any format."""
        out = np.zeros(width, dtype=np.float32)
        if not self.lib.orc_format_row_f32(_ptr(out), qtype, _ptr(data), width, row):
            raise ValueError("unsupported row type")
        return out

    def block_lanes(self, qtype, block, q8k_block):
        """(eight int32 lanes, integer min / correction term) of one super-block."""
        lanes = np.zeros(8, dtype=np.int32)
        extra = ctypes.c_int32(0)
        if not self.lib.orc_format_block_lanes(qtype, _ptr(block), _ptr(q8k_block), _ptr(lanes), ctypes.byref(extra)):
            raise ValueError("not a Q8_K-path format")
        return lanes, extra.value

    def block_decode(self, qtype, block):
        """(q[256], s16[16]) integer weights and 16-element scales."""
        q = np.zeros(256, dtype=np.int32)
        s16 = np.zeros(16, dtype=np.int32)
        if not self.lib.orc_format_block_decode(qtype, _ptr(block), _ptr(q), _ptr(s16)):
            raise ValueError("not a Q8_K-path format")
        return q, s16

    def gemm(self, qtype, data, rows, q8k, batch):
        out = np.zeros(batch * rows, dtype=np.float32)
        width = q8k.size // batch * 256
        if not self.lib.orc_gemm_q8_k(_ptr(out), _ptr(q8k), batch, width, qtype, _ptr(data), rows):
            raise ValueError("bad GEMM arguments")
        return out.reshape(batch, rows)

    def row_f32(self, qtype, data, width, row):
        out = np.zeros(width, dtype=np.float32)
        if not self.lib.orc_row_f32(_ptr(out), qtype, _ptr(data), width, row):
            raise ValueError("unsupported row type")
        return out

    def argmax(self, values):
        values = np.ascontiguousarray(values, dtype=np.float32)
        return int(self.lib.orc_argmax(_ptr(values), values.size))

    def accept(self, batch_logits, drafts):
        batch_logits = np.ascontiguousarray(batch_logits, dtype=np.float32)
        drafts = np.ascontiguousarray(drafts, dtype=np.uint32)
        rows, count = batch_logits.shape
        matched, nxt = ctypes.c_uint32(), ctypes.c_uint32()
        accepted = np.zeros(rows, dtype=np.uint32)
        consumed = self.lib.orc_accept(_ptr(batch_logits), rows, count, _ptr(drafts),
                                       ctypes.byref(matched), ctypes.byref(nxt), _ptr(accepted))
        return int(consumed), int(matched.value), int(nxt.value), accepted[:consumed].copy()

    def sample(self, logits, state, temperature, top_p, presence_penalty, top_k, presence=None):
        """orc_sample: (token, state after the call)."""
        logits, presence = _sample_args(logits, presence)
        token = np.zeros(1, dtype=np.uint32)
        st = ctypes.c_uint64(state)
        if not self.lib.orc_sample(_ptr(token), ctypes.byref(st), _ptr(logits), logits.size, temperature, top_p,
                                   presence_penalty, top_k, None if presence is None else _ptr(presence),
                                   0 if presence is None else presence.size):
            raise ValueError("orc_sample refused its arguments")
        return int(token[0]), st.value

    def grid_entry(self, index):
        out = np.zeros(8, dtype=np.int8)
        self.lib.orc_iq1m_grid_entry(index, _ptr(out))
        return out

    def attention_decode(self, q_and_gate, key, value, key_cache, value_cache, q_norm, k_norm, position):
        """Returns the gated attention output [6144]; updates the caches in place."""
        out = np.zeros(6144, dtype=np.float32)
        args = [np.ascontiguousarray(a, dtype=np.float32) for a in (q_and_gate, key, value, q_norm, k_norm)]
        assert key_cache.dtype == np.float32 and value_cache.dtype == np.float32
        self.lib.orc_attention_decode(_ptr(out), _ptr(args[0]), _ptr(args[1]), _ptr(args[2]),
                                      _ptr(key_cache), _ptr(value_cache), _ptr(args[3]), _ptr(args[4]),
                                      position)
        return out


class Reference:
    """The reference's compiled C kernels (oracle/_ref), when present."""

    def __init__(self, path=REF_SO):
        if not os.path.exists(path):
            raise RuntimeError("reference library not built (oracle/_ref)")
        lib = ctypes.CDLL(path)
        lib.q38_f16_to_f32.restype = ctypes.c_float
        lib.q38_f16_to_f32.argtypes = [ctypes.c_uint16]
        lib.q38_quantize_q8_k.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_uint64]
        lib.q38_tensor_gemv_q8_k.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_uint64,
                                             ctypes.POINTER(GGUFTensor)]
        lib.q38_tensor_gemm_q8_k.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_uint32,
                                             ctypes.c_uint64, ctypes.POINTER(GGUFTensor)]
        lib.q38_tensor_row_f32.argtypes = [ctypes.c_void_p, ctypes.POINTER(GGUFTensor), ctypes.c_uint64]
        lib.q38_tensor_gemv_f32.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.POINTER(GGUFTensor)]
        lib.q38_tensor_gemm_f32.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_uint32, ctypes.c_uint64,
                                            ctypes.POINTER(GGUFTensor)]
        lib.q38ref_full_core.argtypes = [ctypes.c_void_p] * 6 + [ctypes.c_uint32, ctypes.c_void_p,
                                                                  ctypes.c_void_p, ctypes.c_uint32]
        lib.q38_sampler_init.argtypes = [ctypes.POINTER(Q38Sampler), ctypes.c_uint64]
        lib.q38_sample.argtypes = [ctypes.POINTER(Q38Sampler), ctypes.c_void_p, ctypes.c_uint32, ctypes.c_void_p]
        self.lib = lib

    @staticmethod
    def available(path=REF_SO):
        return os.path.exists(path)

    def f16_to_f32(self, bits):
        return self.lib.q38_f16_to_f32(int(bits))

    def quantize(self, x):
        x = np.ascontiguousarray(x, dtype=np.float32)
        out = np.zeros(x.size // 256, dtype=Q8K_DTYPE)
        if not self.lib.q38_quantize_q8_k(_ptr(out), _ptr(x), x.size):
            raise ValueError("length must be a multiple of 256")
        return out

    def gemv(self, qtype, data, rows, q8k):
        width = q8k.size * 256
        tensor = make_tensor(data, qtype, width, rows)
        out = np.zeros(rows, dtype=np.float32)
        if not self.lib.q38_tensor_gemv_q8_k(_ptr(out), _ptr(q8k), width, ctypes.byref(tensor)):
            raise ValueError("bad GEMV arguments")
        return out

    def gemm(self, qtype, data, rows, q8k, batch):
        width = q8k.size // batch * 256
        tensor = make_tensor(data, qtype, width, rows)
        out = np.zeros(batch * rows, dtype=np.float32)
        if not self.lib.q38_tensor_gemm_q8_k(_ptr(out), _ptr(q8k), batch, width, ctypes.byref(tensor)):
            raise ValueError("bad GEMM arguments")
        return out.reshape(batch, rows)

    def gemv_f32(self, qtype, data, rows, x):
        x = np.ascontiguousarray(x, dtype=np.float32)
        tensor = make_tensor(data, qtype, x.size, rows)
        out = np.zeros(rows, dtype=np.float32)
        if not self.lib.q38_tensor_gemv_f32(_ptr(out), _ptr(x), ctypes.byref(tensor)):
            raise ValueError("bad float GEMV arguments")
        return out

    def gemm_f32(self, qtype, data, rows, x):
        """x: [batch, width] fp32 -> [batch, rows]"""
        x = np.ascontiguousarray(x, dtype=np.float32)
        batch, width = x.shape
        tensor = make_tensor(data, qtype, width, rows)
        out = np.zeros(batch * rows, dtype=np.float32)
        if not self.lib.q38_tensor_gemm_f32(_ptr(out), _ptr(x), batch, width, ctypes.byref(tensor)):
            raise ValueError("bad float GEMM arguments")
        return out.reshape(batch, rows)

    def row_f32(self, qtype, data, width, row, rows):
        tensor = make_tensor(data, qtype, width, rows)
        out = np.zeros(width, dtype=np.float32)
        if not self.lib.q38_tensor_row_f32(_ptr(out), ctypes.byref(tensor), row):
            raise ValueError("row decode failed")
        return out


    def sampler_init(self, seed):
        """q38_sampler_init (qwen38_sampler.c:22-32) -> the Q38Sampler fields."""
        sampler = Q38Sampler()
        self.lib.q38_sampler_init(ctypes.byref(sampler), seed)
        return {f: getattr(sampler, f) for f in ("state", "temperature", "top_p", "presence_penalty", "top_k")}

    def sample(self, logits, state, temperature, top_p, presence_penalty, top_k, presence=None):
        """q38_sample (qwen38_sampler.c:51-119): (token, state after the call)."""
        logits, presence = _sample_args(logits, presence)
        sampler = Q38Sampler(state, temperature, top_p, presence_penalty, top_k,
                             None if presence is None else presence.ctypes.data,
                             0 if presence is None else presence.size)
        token = np.zeros(1, dtype=np.uint32)
        if not self.lib.q38_sample(ctypes.byref(sampler), _ptr(logits), logits.size, _ptr(token)):
            raise ValueError("q38_sample refused its arguments")
        return int(token[0]), sampler.state

    def full_core(self, q_and_gate, key, value, key_cache, value_cache, q_norm, k_norm, position):
        """The reference's static q38_full_core (qwen38_model.c:816-885)
        through oracle/ref_attention_shim.c: the gated attention output
        [6144] of one row; key_cache / value_cache ([context, 1024] fp32)
        are updated in place."""
        out = np.zeros(6144, dtype=np.float32)
        args = [np.ascontiguousarray(a, dtype=np.float32).copy() for a in (q_and_gate, key, value, q_norm, k_norm)]
        assert key_cache.dtype == np.float32 and value_cache.dtype == np.float32
        assert key_cache.flags.c_contiguous and value_cache.flags.c_contiguous
        if not self.lib.q38ref_full_core(_ptr(out), _ptr(args[0]), _ptr(args[1]), _ptr(args[2]), _ptr(key_cache),
                                         _ptr(value_cache), key_cache.shape[0], _ptr(args[3]), _ptr(args[4]),
                                         position):
            raise ValueError("q38ref_full_core refused its arguments")
        return out


class ModelAPI:
    """The engine ABI of include/qwen38/qwen38_model.h:10-50 over any library
    that exports it (the compiled reference in oracle/_ref, or libq38hip)."""

    VOCAB = 248320
    HIDDEN = 5120

    def __init__(self, lib):
        lib.q38_model_open_gguf.restype = ctypes.c_void_p
        lib.q38_model_open_gguf.argtypes = [ctypes.c_char_p, ctypes.c_uint32]
        lib.q38_model_attach_mtp_gguf.argtypes = [ctypes.c_void_p, ctypes.c_char_p]
        lib.q38_model_close.argtypes = [ctypes.c_void_p]
        lib.q38_model_reset.argtypes = [ctypes.c_void_p]
        lib.q38_model_forward_token.argtypes = [ctypes.c_void_p, ctypes.c_uint32, ctypes.POINTER(_f32p)]
        lib.q38_model_prefill.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_uint32, ctypes.POINTER(_f32p)]
        lib.q38_model_enable_mtp.argtypes = [ctypes.c_void_p]
        lib.q38_model_mtp_forward.argtypes = [ctypes.c_void_p, ctypes.c_uint32, ctypes.POINTER(_f32p)]
        lib.q38_model_speculative_greedy.argtypes = [ctypes.c_void_p, ctypes.c_uint32, ctypes.c_uint32,
                                                     ctypes.c_uint32, ctypes.c_void_p, _u32p,
                                                     ctypes.POINTER(_f32p)]
        lib.q38_model_forward_token_layers.argtypes = [ctypes.c_void_p, ctypes.c_uint32, ctypes.c_uint32,
                                                       ctypes.c_void_p]
        for name in ("q38_model_vocab_size", "q38_model_position", "q38_model_context_length"):
            getattr(lib, name).restype = ctypes.c_uint32
            getattr(lib, name).argtypes = [ctypes.c_void_p]
        self.lib = lib
        self.handle = None

    def open(self, path, context_length):
        self.handle = self.lib.q38_model_open_gguf(path.encode(), context_length)
        if not self.handle:
            raise RuntimeError("q38_model_open_gguf failed for %s" % path)
        return self

    def close(self):
        if self.handle:
            self.lib.q38_model_close(self.handle)
            self.handle = None

    def _logits(self, pointer):
        return np.ctypeslib.as_array(pointer, shape=(self.VOCAB,)).copy()

    def reset(self):
        self.lib.q38_model_reset(self.handle)

    def attach_mtp(self, path):
        """q38_model_attach_mtp_gguf: the MTP block from a separate GGUF."""
        if not self.lib.q38_model_attach_mtp_gguf(self.handle, path.encode()):
            raise RuntimeError("q38_model_attach_mtp_gguf failed for %s" % path)

    def try_speculative_greedy(self, token, stop_token, draft_count):
        """The raw call: (return value, accepted ids, logits or None).  For
        tests of the failure contract, where 0 is the expected answer."""
        accepted = np.zeros(max(int(draft_count), 1), dtype=np.uint32)
        count = ctypes.c_uint32(0)
        p = _f32p()
        ok = self.lib.q38_model_speculative_greedy(self.handle, int(token), int(stop_token), int(draft_count),
                                                   accepted.ctypes.data, ctypes.byref(count), ctypes.byref(p))
        if not ok:
            return 0, None, None
        return ok, accepted[:count.value].copy(), np.ctypeslib.as_array(p, shape=(248320,)).copy()

    def enable_mtp(self):
        if not self.lib.q38_model_enable_mtp(self.handle):
            raise RuntimeError("q38_model_enable_mtp failed")

    def forward_token(self, token):
        p = _f32p()
        if not self.lib.q38_model_forward_token(self.handle, token, ctypes.byref(p)):
            raise RuntimeError("q38_model_forward_token failed")
        return self._logits(p)

    def prefill(self, tokens):
        tokens = np.ascontiguousarray(tokens, dtype=np.uint32)
        p = _f32p()
        if not self.lib.q38_model_prefill(self.handle, _ptr(tokens), tokens.size, ctypes.byref(p)):
            raise RuntimeError("q38_model_prefill failed")
        return self._logits(p)

    def mtp_forward(self, token):
        p = _f32p()
        if not self.lib.q38_model_mtp_forward(self.handle, token, ctypes.byref(p)):
            raise RuntimeError("q38_model_mtp_forward failed")
        return self._logits(p)

    def speculative_greedy(self, token, stop_token, draft_count):
        accepted = np.zeros(max(draft_count, 1), dtype=np.uint32)
        count = ctypes.c_uint32(0)
        p = _f32p()
        if not self.lib.q38_model_speculative_greedy(self.handle, token, stop_token, draft_count,
                                                     _ptr(accepted), ctypes.byref(count), ctypes.byref(p)):
            raise RuntimeError("q38_model_speculative_greedy failed")
        return accepted[:count.value].copy(), self._logits(p)

    def forward_token_layers(self, token, layers):
        hidden = np.zeros(self.HIDDEN, dtype=np.float32)
        if not self.lib.q38_model_forward_token_layers(self.handle, token, layers, _ptr(hidden)):
            raise RuntimeError("q38_model_forward_token_layers failed")
        return hidden

    def position(self):
        return self.lib.q38_model_position(self.handle)


def reference_model(path=REF_SO):
    """ModelAPI over the compiled reference (oracle/_ref/libq38ref.so)."""
    if not os.path.exists(path):
        raise RuntimeError("reference library not built (oracle/_ref)")
    return ModelAPI(ctypes.CDLL(path))
