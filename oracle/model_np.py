"""CPU restatement of the Qwen3.8 decode block for small cases -- TEST
INFRASTRUCTURE ONLY (tests/ and debugging; the product never imports it).

Reads tensors of a GGUF file by name (numpy memmap) and restates
src/qwen38/qwen38_model.c for ONE token on a fresh state, in float32 numpy
with the reference's operation order (one rounding per operation, the
double-precision squared sums of the norms, and the host C library's expf /
logf through ctypes).  The quantised projections call a `gemv(tensor, x)`
supplied by the caller (the oracle or the compiled reference).
"""
import ctypes
import struct

import numpy as np

_libm = ctypes.CDLL("libm.so.6")
_libm.expf.restype = ctypes.c_float
_libm.expf.argtypes = [ctypes.c_float]
_libm.logf.restype = ctypes.c_float
_libm.logf.argtypes = [ctypes.c_float]

F32 = np.float32
GGML_BLOCK = {0: (1, 4), 12: (256, 144), 14: (256, 210), 29: (256, 56)}


def expf(v):
    return F32(_libm.expf(float(v)))


def logf(v):
    return F32(_libm.logf(float(v)))


class GGUF:
    """Minimal GGUF v3 reader: tensor name -> (type, shape, bytes)."""

    def __init__(self, path):
        self.path = path
        self.mm = np.memmap(path, dtype=np.uint8, mode="r")
        buf = self.mm
        pos = 0

        def take(fmt):
            nonlocal pos
            size = struct.calcsize(fmt)
            out = struct.unpack_from(fmt, buf, pos)
            pos += size
            return out

        def string():
            nonlocal pos
            (n,) = take("<Q")
            s = bytes(buf[pos:pos + n]).decode()
            pos += n
            return s

        sizes = {0: 1, 1: 1, 2: 2, 3: 2, 4: 4, 5: 4, 6: 4, 7: 1, 10: 8, 11: 8, 12: 8}
        magic, version, n_tensors, n_kv = take("<IIQQ")
        assert magic == 0x46554747 and version in (2, 3)
        self.meta = {}
        for _ in range(n_kv):
            key = string()
            (vt,) = take("<I")
            if vt == 8:
                self.meta[key] = string()
            elif vt == 9:
                at, count = take("<IQ")
                for _ in range(count):
                    if at == 8:
                        string()
                    else:
                        pos += sizes[at]
            else:
                raw = bytes(buf[pos:pos + sizes[vt]])
                pos += sizes[vt]
                self.meta[key] = int.from_bytes(raw, "little")
        infos = {}
        for _ in range(n_tensors):
            name = string()
            (nd,) = take("<I")
            shape = take("<%dQ" % nd)
            ttype, offset = take("<IQ")
            infos[name] = (ttype, shape, offset)
        align = self.meta.get("general.alignment", 32)
        data = (pos + align - 1) // align * align
        self.tensors = {}
        for name, (ttype, shape, offset) in infos.items():
            be, bb = GGML_BLOCK[ttype]
            n = int(np.prod(shape)) // be * bb
            self.tensors[name] = (ttype, shape, data + offset, n)

    def raw(self, name):
        ttype, shape, start, n = self.tensors[name]
        return ttype, shape, self.mm[start:start + n]

    def f32(self, name):
        ttype, shape, data = self.raw(name)
        assert ttype == 0
        return np.frombuffer(data, dtype=np.float32)


def rmsnorm(x, w):
    """q38_rmsnorm (qwen38_model.c:426-435)"""
    s = 0.0
    for v in (x * x).astype(np.float32):
        s += float(v)
    mean = F32(s / float(x.size))
    scale = F32(1.0) / np.sqrt(mean + F32(1e-6), dtype=np.float32)
    return (x * scale).astype(np.float32) * w


def l2norm(x):
    """q38_l2norm (:608-614)"""
    s = 0.0
    for v in (x * x).astype(np.float32):
        s += float(v)
    scale = F32(1.0) / np.maximum(np.sqrt(F32(s), dtype=np.float32), F32(1e-6))
    return x * scale


def sigmoid(v):
    return F32(1.0) / (F32(1.0) + expf(-v))


def silu(v):
    return F32(v) / (F32(1.0) + expf(-F32(v)))


def softplus(v):
    if v > F32(20.0):
        return F32(v)
    return logf(F32(1.0) + expf(v))


def avx2_dot128(products_fma_chain):
    """reduction of q38_dot_f32_128 (:616-637) over 32 per-lane accumulators"""
    p = products_fma_chain
    q = [(p[j] + p[16 + j]) + (p[8 + j] + p[24 + j]) for j in range(8)]
    h = [q[j] + q[j + 4] for j in range(4)]
    return (h[0] + h[1]) + (h[2] + h[3])


def fma32(a, b, c):
    """exact fmaf via float64 (a*b exact in double; one rounding of the sum
    is not guaranteed in double, so use the exact rational form)"""
    from fractions import Fraction
    r = Fraction(float(a)) * Fraction(float(b)) + Fraction(float(c))
    return F32(float(r)) if True else None


def deltanet_first_token(g, layer, hidden_norm, gemv):
    """q38_linear_attention + q38_linear_core (:720-812) for the first token
    (zero conv and delta state).  Returns dict of intermediates."""
    p = "blk.%d." % layer
    qkv = gemv(p + "attn_qkv.weight", hidden_norm)
    z = gemv(p + "attn_gate.weight", hidden_norm)
    beta = gemv(p + "ssm_beta.weight", hidden_norm)
    alpha = gemv(p + "ssm_alpha.weight", hidden_norm)
    out = {"qkv_proj": qkv.copy(), "z": z.copy(), "beta_proj": beta.copy(), "alpha_proj": alpha.copy()}
    conv = g.f32(p + "ssm_conv1d.weight").reshape(10240, 4)
    conv_out = np.empty(10240, np.float32)
    for ch in range(10240):
        value = F32(0.0)
        value = value + F32(0.0) * conv[ch, 0]
        value = value + F32(0.0) * conv[ch, 1]
        value = value + F32(0.0) * conv[ch, 2]
        value = value + qkv[ch] * conv[ch, 3]
        conv_out[ch] = value
    act = np.array([silu(v) for v in conv_out], np.float32)
    out["conv_silu"] = act.copy()
    q = act[:2048].copy()
    k = act[2048:4096].copy()
    v = act[4096:]
    for h in range(16):
        q[h * 128:(h + 1) * 128] = l2norm(q[h * 128:(h + 1) * 128])
        k[h * 128:(h + 1) * 128] = l2norm(k[h * 128:(h + 1) * 128])
    a = g.f32(p + "ssm_a")
    dt = g.f32(p + "ssm_dt.bias")
    beta_t = np.array([sigmoid(b) for b in beta], np.float32)
    alpha_t = np.array([a[h] * softplus(alpha[h] + dt[h]) for h in range(48)], np.float32)
    out["beta"], out["alpha"] = beta_t, alpha_t
    query_scale = F32(1.0) / np.sqrt(F32(128.0), dtype=np.float32)
    attn = np.empty(6144, np.float32)
    for vh in range(48):
        kh = vh % 16
        qv, kv = q[kh * 128:(kh + 1) * 128], k[kh * 128:(kh + 1) * 128]
        for c in range(128):
            delta = (v[vh * 128 + c] - F32(0.0)) * beta_t[vh]
            upd = np.array([fma32(kv[e], delta, F32(0.0)) for e in range(128)], np.float32)
            acc = []
            for lane in range(32):
                s = F32(0.0)
                for i4 in range(4):
                    s = fma32(upd[32 * i4 + lane], qv[32 * i4 + lane], s)
                acc.append(s)
            attn[vh * 128 + c] = avx2_dot128(acc) * query_scale
    out["core"] = attn.copy()
    nw = g.f32(p + "ssm_norm.weight")
    for vh in range(48):
        seg = rmsnorm(attn[vh * 128:(vh + 1) * 128], nw)
        gate = z[vh * 128:(vh + 1) * 128]
        attn[vh * 128:(vh + 1) * 128] = np.array([seg[i] * silu(gate[i]) for i in range(128)], np.float32)
    out["gated"] = attn
    return out
