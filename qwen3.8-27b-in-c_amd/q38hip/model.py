"""ctypes mirror of the model ABI (include/q38model.h), which keeps the names
and semantics of the reference engine's include/qwen38/qwen38_model.h.

    m = Model.open("model.gguf", context_length=1024)
    m.enable_mtp()
    logits = m.prefill(prompt)            # numpy float32[248320] copy
    accepted, logits = m.speculative_greedy(token, stop, 3)

Every call runs the HIP kernels of libq38hip.so on the model's own stream
and returns after the results are on the host.
"""
import ctypes

import numpy as np

from . import LIB_PATH, load_library

VOCAB = 248320
HIDDEN = 5120
_f32p = ctypes.POINTER(ctypes.c_float)
_u32p = ctypes.POINTER(ctypes.c_uint32)


def _bind(lib):
    vp, u32 = ctypes.c_void_p, ctypes.c_uint32
    lib.q38_model_open_gguf.restype = vp
    lib.q38_model_open_gguf.argtypes = [ctypes.c_char_p, u32]
    lib.q38_model_attach_mtp_gguf.argtypes = [vp, ctypes.c_char_p]
    lib.q38_model_close.restype = None
    lib.q38_model_close.argtypes = [vp]
    lib.q38_model_reset.restype = None
    lib.q38_model_reset.argtypes = [vp]
    lib.q38_model_forward_token.argtypes = [vp, u32, ctypes.POINTER(_f32p)]
    lib.q38_model_prefill.argtypes = [vp, vp, u32, ctypes.POINTER(_f32p)]
    lib.q38_model_enable_mtp.argtypes = [vp]
    lib.q38_model_mtp_forward.argtypes = [vp, u32, ctypes.POINTER(_f32p)]
    lib.q38_model_speculative_greedy.argtypes = [vp, u32, u32, u32, vp, _u32p, ctypes.POINTER(_f32p)]
    lib.q38_model_forward_token_layers.argtypes = [vp, u32, u32, vp]
    f32, u64p = ctypes.c_float, ctypes.POINTER(ctypes.c_uint64)
    lib.q38hip_model_sample.argtypes = [vp, u64p, f32, f32, f32, u32, vp, u32, _u32p]
    lib.q38hip_model_forward_sample.argtypes = [vp, u32, u64p, f32, f32, f32, u32, vp, u32, _u32p]
    for name in ("q38_model_vocab_size", "q38_model_position", "q38_model_context_length"):
        getattr(lib, name).restype = u32
        getattr(lib, name).argtypes = [vp]
    return lib


class Model:
    def __init__(self, handle, lib):
        self.handle = handle
        self.lib = lib

    @classmethod
    def open(cls, path, context_length, lib_path=LIB_PATH):
        lib = _bind(load_library(lib_path))
        handle = lib.q38_model_open_gguf(path.encode(), context_length)
        if not handle:
            raise RuntimeError("q38_model_open_gguf failed for %s" % path)
        return cls(handle, lib)

    def close(self):
        if self.handle:
            self.lib.q38_model_close(self.handle)
            self.handle = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    @staticmethod
    def _copy(pointer):
        return np.ctypeslib.as_array(pointer, shape=(VOCAB,)).copy()

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
        if not self.lib.q38_model_forward_token(self.handle, int(token), ctypes.byref(p)):
            raise RuntimeError("q38_model_forward_token failed")
        return self._copy(p)

    def prefill(self, tokens):
        tokens = np.ascontiguousarray(tokens, dtype=np.uint32)
        p = _f32p()
        if not self.lib.q38_model_prefill(self.handle, tokens.ctypes.data, tokens.size, ctypes.byref(p)):
            raise RuntimeError("q38_model_prefill failed")
        return self._copy(p)

    def mtp_forward(self, token):
        p = _f32p()
        if not self.lib.q38_model_mtp_forward(self.handle, int(token), ctypes.byref(p)):
            raise RuntimeError("q38_model_mtp_forward failed")
        return self._copy(p)

    def speculative_greedy(self, token, stop_token, draft_count, logits=True):
        """(accepted token ids, logits after the last one); with logits=False
        the second item is None and the library's logits buffer is not copied
        (a caller that only follows the accepted tokens, as the reference's
        CLI loop does)."""
        accepted = np.zeros(max(int(draft_count), 1), dtype=np.uint32)
        count = ctypes.c_uint32(0)
        p = _f32p()
        if not self.lib.q38_model_speculative_greedy(self.handle, int(token), int(stop_token), int(draft_count),
                                                     accepted.ctypes.data, ctypes.byref(count), ctypes.byref(p)):
            raise RuntimeError("q38_model_speculative_greedy failed")
        return accepted[:count.value].copy(), (self._copy(p) if logits else None)

    @staticmethod
    def _sampler_args(sampler):
        presence = sampler.presence
        if presence is not None:
            if not (isinstance(presence, np.ndarray) and presence.dtype == np.uint8 and presence.flags.c_contiguous):
                raise ValueError("presence must be a contiguous numpy uint8 array")
        return (sampler.temperature, sampler.top_p, sampler.presence_penalty, sampler.top_k,
                None if presence is None else presence.ctypes.data, 0 if presence is None else presence.size)

    def sample(self, sampler):
        """q38hip_model_sample: q38_sample over the last returned logits, on
        the device; sampler.state advances.  Returns the token id."""
        state = ctypes.c_uint64(sampler.state)
        token = ctypes.c_uint32(0)
        if not self.lib.q38hip_model_sample(self.handle, ctypes.byref(state), *self._sampler_args(sampler),
                                            ctypes.byref(token)):
            raise RuntimeError("q38hip_model_sample failed")
        sampler.state = state.value
        return token.value

    def forward_sample(self, token, sampler):
        """q38hip_model_forward_sample: forward_token(token) then sample,
        without downloading the logits.  Returns the sampled token id."""
        state = ctypes.c_uint64(sampler.state)
        out = ctypes.c_uint32(0)
        if not self.lib.q38hip_model_forward_sample(self.handle, int(token), ctypes.byref(state),
                                                    *self._sampler_args(sampler), ctypes.byref(out)):
            raise RuntimeError("q38hip_model_forward_sample failed")
        sampler.state = state.value
        return out.value

    def forward_token_layers(self, token, layers):
        hidden = np.zeros(HIDDEN, dtype=np.float32)
        if not self.lib.q38_model_forward_token_layers(self.handle, int(token), int(layers), hidden.ctypes.data):
            raise RuntimeError("q38_model_forward_token_layers failed")
        return hidden

    def position(self):
        return self.lib.q38_model_position(self.handle)

    def context_length(self):
        return self.lib.q38_model_context_length(self.handle)
