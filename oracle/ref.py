"""numpy front end over liboracle.so, the C restatement in afref.c.

TEST INFRASTRUCTURE ONLY: the checker the parity tests, smoke() and bench.py's
CPU-baseline leg compare the HIP library against. Every function names the
reference file:line it restates; the C source carries the same citations.

Parity-pin status of each function (what checks it independently of itself)
is listed in PINS below and asserted by tests/test_oracle.py.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liboracle.so")

# What pins each oracle function (see tests/test_oracle.py).
PINS = {
    "f32_to_f16": "reference KATs test/float16.test.ts:5-33; numpy IEEE RNE over all normal-range results",
    "f16_to_f32": "reference KATs test/dtype.test.ts:6-11; numpy float16 decode over all 65536 bit patterns",
    "q8_block_decode": "reference KAT test/dtype.test.ts:13-23",
    "q8_block_encode": "round trip |w - decode(encode(w))| <= scale/2 and max code 127 per block",
    "q8_channel_decode": "closed form f32(q)*s (single rounded product) vs numpy float32 multiply",
    "gemm_f64": "numpy float64 matmul",
    "linear": "numpy float64 matmul + bias + relu",
    "attention_project": "numpy float64 closed form",
    "triangle_outgoing": "reference fixtures openfold-triangle-small, AlphaFold short-9 (and the two "
                         "59-residue fixtures when /root/reference is present)",
    "triangle_incoming": "identity incoming(z) = T(outgoing(T(z))) with T the pair transpose, over every "
                         "outgoing fixture; numpy einsum 'kjc,kic->ijc' restatement",
    "opm": "numpy float64 restatement of AlphaFold's OuterProductMean; closed forms (rank one, all-ones "
           "mask count = S)",
    "transition": "numpy float64 restatement; closed form with ReLU inactive",
    "attention": "closed forms: a fully masked row averages v (the logit clamp), a one-hot pair bias "
                 "selects one key, zero query weights give uniform weights; transpose equivalence; a "
                 "loop-over-keys restatement with an explicit running softmax at small sizes",
}


def _build() -> None:
    subprocess.run(["make", "-s", "-C", _HERE, "liboracle.so"], check=True)


def _load() -> ctypes.CDLL:
    if not os.path.exists(_LIB_PATH):
        _build()
    return ctypes.CDLL(_LIB_PATH)


_lib = _load()

_f32p = np.ctypeslib.ndpointer(np.float32, flags="C_CONTIGUOUS")
_f64p = np.ctypeslib.ndpointer(np.float64, flags="C_CONTIGUOUS")
_u16p = np.ctypeslib.ndpointer(np.uint16, flags="C_CONTIGUOUS")
_i8p = np.ctypeslib.ndpointer(np.int8, flags="C_CONTIGUOUS")
_sz = ctypes.c_size_t


def _sig(name, res, args):
    fn = getattr(_lib, name)
    fn.restype = res
    fn.argtypes = args
    return fn


_f32_to_f16 = _sig("afref_f32_to_f16_array", None, [_f32p, _u16p, _sz])
_f16_to_f32 = _sig("afref_f16_to_f32_array", None, [_u16p, _f32p, _sz])
_q8_encode = _sig("afref_q8_block_encode", None, [_f32p, _sz, ctypes.c_int, _i8p, _u16p])
_q8_decode = _sig("afref_q8_block_decode", None, [_i8p, _u16p, ctypes.c_int, _sz, _sz, _f32p])
_q8_channel = _sig("afref_q8_channel_decode", None, [_i8p, _f32p, ctypes.c_int, ctypes.c_int, _f32p])
_normal = _sig("afref_normal_f32", None, [ctypes.c_uint64, ctypes.c_double, ctypes.c_double, _sz, _f32p])
_uniform = _sig("afref_uniform_f32", None, [ctypes.c_uint64, ctypes.c_double, ctypes.c_double, _sz, _f32p])
_uniform_i8 = _sig("afref_uniform_i8", None, [ctypes.c_uint64, ctypes.c_int, ctypes.c_int, _sz, _i8p])
_mulberry = _sig("afref_mulberry_uniform", None, [ctypes.c_uint32, _sz, _f64p])
_lcg = _sig("afref_lcg_values", None, [ctypes.c_uint32, _sz, _f32p])
_gemm_f64 = _sig("afref_gemm_f64", None, [_f32p, _f32p, ctypes.c_void_p, ctypes.c_int, ctypes.c_int,
                                          ctypes.c_int, _f64p])
_linear = _sig("afref_linear", None, [_f32p, _f32p, ctypes.c_void_p, ctypes.c_int, ctypes.c_int,
                                      ctypes.c_int, ctypes.c_int, ctypes.c_int, _f32p])
_attn = _sig("afref_attention_project", None, [_f32p, _f32p, ctypes.c_void_p, ctypes.c_int, ctypes.c_int,
                                               ctypes.c_int, ctypes.c_int, _f32p, _f32p, _f32p, _f32p])
_tri = _sig("afref_triangle", None, [ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int, _f32p, _f32p,
                                     _f32p, ctypes.c_double, _f32p])
_opm = _sig("afref_opm", None, [ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int, _f32p,
                                _f32p, _f32p, ctypes.c_double, ctypes.c_double, _f32p])
_transition = _sig("afref_transition", None, [_sz, ctypes.c_int, ctypes.c_int, _f32p, _f32p,
                                              ctypes.c_double, _f32p])
_set_threads = _sig("afref_set_threads", None, [ctypes.c_int])
_max_threads = _sig("afref_max_threads", ctypes.c_int, [])


def set_threads(threads: int) -> None:
    """OpenMP threads of the triangle's loops (same bits at any count)."""
    _set_threads(int(threads))


def max_threads() -> int:
    return int(_max_threads())


def _c32(x) -> np.ndarray:
    return np.ascontiguousarray(x, dtype=np.float32)


def _ptr(x):
    return None if x is None else x.ctypes.data_as(ctypes.c_void_p)


# --- f16 and int8 codecs ---------------------------------------------------

def f32_to_f16(values) -> np.ndarray:
    """src/runtime/float16.ts:5-35 — bit patterns as uint16."""
    v = _c32(values)
    out = np.empty(v.shape, np.uint16)
    _f32_to_f16(v.reshape(-1), out.reshape(-1), v.size)
    return out


def f16_to_f32(bits) -> np.ndarray:
    """src/reference/dtype.ts:28-35."""
    b = np.ascontiguousarray(bits, dtype=np.uint16)
    out = np.empty(b.shape, np.float32)
    _f16_to_f32(b.reshape(-1), out.reshape(-1), b.size)
    return out


def round_f16(values) -> np.ndarray:
    """f32 values rounded through the reference's f16 encoder, back as f32."""
    return f16_to_f32(f32_to_f16(values))


def q8_block_encode(values, block: int = 64):
    """tools/quantize-web-model.ts:98-119 — (codes int8, scales f16 bits)."""
    v = _c32(values).reshape(-1)
    codes = np.empty(v.size, np.int8)
    scales = np.empty((v.size + block - 1) // block, np.uint16)
    _q8_encode(v, v.size, block, codes, scales)
    return codes, scales


def q8_block_decode(codes, scales, block: int = 64, start: int = 0, count: int | None = None) -> np.ndarray:
    """src/reference/dtype.ts:66-99 (int8 branch of readTensorRange)."""
    c = np.ascontiguousarray(codes, dtype=np.int8).reshape(-1)
    s = np.ascontiguousarray(scales, dtype=np.uint16).reshape(-1)
    if count is None:
        count = c.size - start
    if start < 0 or count < 0 or start + count > c.size:
        raise ValueError("tensor range is out of bounds")
    out = np.empty(count, np.float32)
    _q8_decode(c, s, block, start, count, out)
    return out


def q8_channel_decode(q, scale) -> np.ndarray:
    """Per-output-channel dequantisation, w[k][n] = f32(q[k][n]) * scale[n]."""
    qq = np.ascontiguousarray(q, dtype=np.int8)
    K, N = qq.shape
    out = np.empty((K, N), np.float32)
    _q8_channel(qq, _c32(scale), K, N, out)
    return out


# --- seeded inputs ----------------------------------------------------------

def normal(seed: int, shape, variance: float = 1.0, mean: float = 0.0) -> np.ndarray:
    n = int(np.prod(shape))
    out = np.empty(n, np.float32)
    _normal(seed, mean, variance, n, out)
    return out.reshape(shape)


def uniform(seed: int, shape, low: float, high: float) -> np.ndarray:
    n = int(np.prod(shape))
    out = np.empty(n, np.float32)
    _uniform(seed, low, high, n, out)
    return out.reshape(shape)


def uniform_i8(seed: int, shape, low: int = -127, high: int = 127) -> np.ndarray:
    n = int(np.prod(shape))
    out = np.empty(n, np.int8)
    _uniform_i8(seed, low, high, n, out)
    return out.reshape(shape)


def mulberry_uniform(seed: int, count: int) -> np.ndarray:
    """src/testing/deterministic-input.ts:7-16."""
    out = np.empty(count, np.float64)
    _mulberry(seed, count, out)
    return out


def lcg_values(seed: int, count: int) -> np.ndarray:
    """test/gemm-half-precision.gpu.test.ts:44-50."""
    out = np.empty(count, np.float32)
    _lcg(seed, count, out)
    return out


TRIANGLE_ORDER = (
    "layerNormInWeight", "layerNormInBias",
    "linearAPWeight", "linearAPBias", "linearAGWeight", "linearAGBias",
    "linearBPWeight", "linearBPBias", "linearBGWeight", "linearBGBias",
    "layerNormOutWeight", "layerNormOutBias",
    "linearZWeight", "linearZBias", "linearGWeight", "linearGBias",
)


def triangle_weight_shapes(cz: int, ch: int) -> dict:
    """src/triangle/types.ts:68-83 — [out][in] weight shapes."""
    return {
        "layerNormInWeight": (cz,), "layerNormInBias": (cz,),
        "linearAPWeight": (ch, cz), "linearAPBias": (ch,),
        "linearAGWeight": (ch, cz), "linearAGBias": (ch,),
        "linearBPWeight": (ch, cz), "linearBPBias": (ch,),
        "linearBGWeight": (ch, cz), "linearBGBias": (ch,),
        "layerNormOutWeight": (ch,), "layerNormOutBias": (ch,),
        "linearZWeight": (cz, ch), "linearZBias": (cz,),
        "linearGWeight": (cz, cz), "linearGBias": (cz,),
    }


def deterministic_triangle_input(length: int, cz: int, ch: int, seed: int = 7) -> dict:
    """src/testing/deterministic-input.ts:18-51 (createDeterministicTriangleInput)."""
    pairs = length * length
    sizes = [cz, cz, ch * cz, ch, ch * cz, ch, ch * cz, ch, ch * cz, ch, ch, ch, cz * ch, cz, cz * cz, cz]
    specs = [(0.1, 1), (0.05, 0), (0.15 / np.sqrt(cz), 0), (0.03, 0), (0.15 / np.sqrt(cz), 0), (0.03, 1),
             (0.15 / np.sqrt(cz), 0), (0.03, 0), (0.15 / np.sqrt(cz), 0), (0.03, 1), (0.1, 1), (0.05, 0),
             (0.15 / np.sqrt(ch), 0), (0.03, 0), (0.15 / np.sqrt(cz), 0), (0.03, 1)]
    total = sum(sizes) + pairs + pairs * cz
    r = mulberry_uniform(seed, total)
    at = 0
    weights = {}
    shapes = triangle_weight_shapes(cz, ch)
    for name, size, (scale, center) in zip(TRIANGLE_ORDER, sizes, specs):
        weights[name] = (center + (r[at:at + size] * 2 - 1) * scale).astype(np.float32).reshape(shapes[name])
        at += size
    mask = (r[at:at + pairs] > 0.15).astype(np.float32).reshape(length, length)
    at += pairs
    z = (0 + (r[at:at + pairs * cz] * 2 - 1) * 1).astype(np.float32).reshape(length, length, cz)
    return {"shape": (length, cz, ch), "z": z, "mask": mask, "weights": weights, "epsilon": 1e-5}


def triangle_pairs(direction: str, z, mask, weights: dict, pairs, epsilon: float = 1e-5) -> np.ndarray:
    """out[i, j, :] of the triangle multiplication for the listed (i, j)
    only, in float64: src/triangle/cpu-reference.ts:6-100 (LayerNorm with
    the biased variance, weights [out][in], gate from the normalised pair),
    the incoming direction contracting over the first index
    (src/triangle/shaders.ts:452-495). Output pair (i, j) reads z's rows i and
    j (outgoing: sum_k a[i,k] b[j,k]) or columns i and j (incoming:
    sum_k a[k,j] b[k,i]) and z[i, j] itself, so a sample of pairs at full
    size costs O(rows * L * c_z * c_h). Returns
    [len(pairs)][c_z]."""
    # Only the rows (outgoing) or columns (incoming) the pairs read are
    # widened to float64, so z may be any size that fits in memory as given.
    m64 = np.asarray(mask, np.float64)
    w = {k: np.asarray(v, np.float64) for k, v in weights.items()}

    def ln(x, g, b):
        mean = x.mean(-1, keepdims=True)
        var = ((x - mean) ** 2).mean(-1, keepdims=True)
        return (x - mean) / np.sqrt(var + epsilon) * g + b

    def sig(x):
        return 1.0 / (1.0 + np.exp(-x))

    projected = {}
    for r in sorted({int(i) for i, _ in pairs} | {int(j) for _, j in pairs}):
        line = np.asarray(z[r] if direction == "outgoing" else z[:, r], np.float64)
        keep = (m64[r] if direction == "outgoing" else m64[:, r])[:, None]
        zn = ln(line, w["layerNormInWeight"], w["layerNormInBias"])
        a = keep * (zn @ w["linearAPWeight"].T + w["linearAPBias"]) * sig(zn @ w["linearAGWeight"].T + w["linearAGBias"])
        b = keep * (zn @ w["linearBPWeight"].T + w["linearBPBias"]) * sig(zn @ w["linearBGWeight"].T + w["linearBGBias"])
        projected[r] = (a, b)
    out = np.empty((len(pairs), z.shape[2]))
    for n, (i, j) in enumerate(pairs):
        # outgoing ikc,jkc->ijc; incoming kjc,kic->ijc (a follows j, b follows i)
        if direction == "outgoing":
            x = (projected[int(i)][0] * projected[int(j)][1]).sum(0)
        else:
            x = (projected[int(j)][0] * projected[int(i)][1]).sum(0)
        x = ln(x, w["layerNormOutWeight"], w["layerNormOutBias"])
        gate = sig(ln(np.asarray(z[i, j], np.float64), w["layerNormInWeight"], w["layerNormInBias"]) @ w["linearGWeight"].T
                   + w["linearGBias"])
        out[n] = (x @ w["linearZWeight"].T + w["linearZBias"]) * gate
    return out


def pack_triangle_weights(weights: dict) -> np.ndarray:
    """src/triangle/weights.ts:20-34 (packWeights, f32)."""
    return np.concatenate([_c32(weights[n]).reshape(-1) for n in TRIANGLE_ORDER])


# --- GEMMs ------------------------------------------------------------------

def gemm_f64(a, w, bias=None) -> np.ndarray:
    """test/gemm-half-precision.gpu.test.ts:52-68."""
    a = _c32(a)
    w = _c32(w)
    M, K = a.shape
    N = w.shape[1]
    out = np.empty((M, N), np.float64)
    b = None if bias is None else _c32(bias)
    _gemm_f64(a, w, _ptr(b), M, K, N, out)
    return out


def linear(a, w, bias=None, relu: bool = False, residual=None) -> np.ndarray:
    """src/evoformer/transition.ts:91-138 (createLinearShader)."""
    a = _c32(a)
    w = _c32(w)
    M, K = a.shape
    N = w.shape[1]
    out = np.zeros((M, N), np.float32) if residual is None else _c32(residual).copy()
    b = None if bias is None else _c32(bias)
    _linear(a, w, _ptr(b), M, K, N, int(relu), int(residual is not None), out)
    return out


def attention_project(x, w, gate_bias, heads: int, head_dim: int):
    """src/evoformer/attention.ts:497-589 — returns (q, k, v, g)."""
    x = _c32(x)
    w = _c32(w)
    M, K = x.shape
    HD = heads * head_dim
    assert w.shape == (K, 4 * HD)
    outs = [np.empty((M, HD), np.float32) for _ in range(4)]
    gb = None if gate_bias is None else _c32(gate_bias)
    _attn(x, w, _ptr(gb), M, K, HD, head_dim, *outs)
    return tuple(outs)


# --- fused operators --------------------------------------------------------

def triangle(direction: str, z, mask, weights: dict, epsilon: float = 1e-5) -> np.ndarray:
    """src/triangle/cpu-reference.ts:56-100 (outgoing); shaders.ts:452-495 (incoming)."""
    z = _c32(z)
    L, L2, cz = z.shape
    assert L == L2
    ch = np.asarray(weights["linearAPBias"]).shape[0]
    packed = pack_triangle_weights(weights)
    out = np.empty((L, L, cz), np.float32)
    _tri(0 if direction == "outgoing" else 1, L, cz, ch, z, _c32(mask), packed, float(epsilon), out)
    return out


OPM_ORDER = ("layerNormScale", "layerNormOffset", "leftWeight", "leftBias", "rightWeight", "rightBias",
             "outputWeight", "outputBias")


def opm(activations, mask, weights: dict, ln_epsilon: float = 1e-5, norm_epsilon: float = 1e-3) -> np.ndarray:
    """test/outer-product-mean-reference.gpu.test.ts:22-78."""
    act = _c32(activations)
    S, L, cm = act.shape
    co = np.asarray(weights["leftBias"]).shape[0]
    cz = np.asarray(weights["outputBias"]).shape[0]
    packed = np.concatenate([_c32(weights[n]).reshape(-1) for n in OPM_ORDER])
    out = np.empty((L, L, cz), np.float32)
    _opm(S, L, cm, co, cz, act, _c32(mask), packed, float(ln_epsilon), float(norm_epsilon), out)
    return out


TRANSITION_ORDER = ("layerNormScale", "layerNormOffset", "firstWeight", "firstBias", "secondWeight",
                    "secondBias")


def transition(activations, weights: dict, epsilon: float = 1e-5) -> np.ndarray:
    """src/evoformer/transition.ts:264-361 (TransitionGpu.run)."""
    act = _c32(activations)
    rows, c = act.shape
    h = np.asarray(weights["firstBias"]).shape[0]
    packed = np.concatenate([_c32(weights[n]).reshape(-1) for n in TRANSITION_ORDER])
    out = np.empty((rows, c), np.float32)
    _transition(rows, c, h, act, packed, float(epsilon), out)
    return out


def error_metrics(actual, expected) -> dict:
    """src/triangle/types.ts:91-110 (errorMetrics)."""
    a = np.asarray(actual, np.float64).reshape(-1)
    e = np.asarray(expected, np.float64).reshape(-1)
    if a.size != e.size or a.size == 0:
        raise ValueError("error metrics require equally sized, non-empty arrays")
    d = np.abs(a - e)
    return {"meanAbsoluteError": float(d.mean()), "maxAbsoluteError": float(d.max()),
            "rootMeanSquareError": float(np.sqrt((d * d).mean()))}


# --- attention ----------------------------------------------------------------

ATTENTION_ORDER = ("queryNormScale", "queryNormOffset", "queryWeight", "keyWeight", "valueWeight",
                   "gatingWeight", "gatingBias", "outputWeight", "outputBias")


def pack_attention_weights(weights: dict, pair_bias: dict | None = None) -> np.ndarray:
    """src/evoformer/attention.ts:179-201 (packAttentionWeights): the nine
    tensors, then for a separate pair bias its LayerNorm scale and offset and
    projection, or for a normalized-input bias its projection."""
    tensors = [_c32(weights[n]).reshape(-1) for n in ATTENTION_ORDER]
    if pair_bias is not None:
        if pair_bias["source"] == "separate":
            tensors += [_c32(pair_bias[n]).reshape(-1) for n in ("layerNormScale", "layerNormOffset",
                                                                  "projectionWeight")]
        else:
            tensors.append(_c32(pair_bias["projectionWeight"]).reshape(-1))
    return np.concatenate(tensors)


def _layer_norm64(x, scale, offset, eps):
    """Row LayerNorm, two-pass mean and biased variance, eps inside the root
    (attention.ts:312-324)."""
    mean = x.mean(axis=-1, keepdims=True)
    var = ((x - mean) ** 2).mean(axis=-1, keepdims=True)
    return (x - mean) / np.sqrt(var + eps) * scale + offset


def attention(activations, mask, weights: dict, batch: int, queries: int, channels: int, heads: int,
              transpose: bool = False, pair_bias: dict | None = None, epsilon: float = 1e-5) -> np.ndarray:
    """src/evoformer/attention.ts:1334-1452 (AttentionGpu.run), in float64.

    Rows are taken in attention order: entry (b, q) of the batch is source row
    b * queries + q, or q * batch + b when transposed (:312-317), as is the
    mask (:428-433). LayerNorm with the query norm; q = x_hat Wq / sqrt(d),
    k, v = x_hat Wk, x_hat Wv, g = sigmoid(x_hat Wg + bg) (:497-560, weights
    [in][out]); a pair bias bias[h][q][k] = y[q][k] . Wb[:, h] with y the
    normalised input in attention order (normalized-input, which needs
    batch == queries) or the LayerNormed separate pair activations
    (:631-661, :1378-1420); logits q.k + 1e9 (mask[b][k] - 1) + bias, clamped
    to [-1e8, 1e8], softmax over keys, times the gate (:688-723); then
    y Wo + bo written back in source order (:1261-1316)."""
    B, Q, C, H = batch, queries, channels, heads
    d = C // H
    x = np.asarray(activations, np.float64).reshape(-1)
    m = np.asarray(mask, np.float64).reshape(-1)
    if transpose:
        X = x.reshape(Q, B, C).transpose(1, 0, 2)
        M = m.reshape(Q, B).T
    else:
        X = x.reshape(B, Q, C)
        M = m.reshape(B, Q)
    w = {k: np.asarray(v, np.float64) for k, v in weights.items()}
    Xn = _layer_norm64(X, w["queryNormScale"], w["queryNormOffset"], epsilon)
    q = (Xn @ w["queryWeight"].reshape(C, C)).reshape(B, Q, H, d) / np.sqrt(d)
    k = (Xn @ w["keyWeight"].reshape(C, C)).reshape(B, Q, H, d)
    v = (Xn @ w["valueWeight"].reshape(C, C)).reshape(B, Q, H, d)
    g = 1.0 / (1.0 + np.exp(-(Xn @ w["gatingWeight"].reshape(C, C) + w["gatingBias"]))).reshape(B, Q, H, d)
    logits = np.einsum("bqhd,bkhd->bhqk", q, k) + 1e9 * (M[:, None, None, :] - 1.0)
    if pair_bias is not None:
        if pair_bias["source"] == "separate":
            P = np.asarray(pair_bias["activations"], np.float64)
            Cp = int(pair_bias["channels"])
            P = _layer_norm64(P.reshape(Q, Q, Cp), np.asarray(pair_bias["layerNormScale"], np.float64),
                              np.asarray(pair_bias["layerNormOffset"], np.float64), epsilon)
            Wb = np.asarray(pair_bias["projectionWeight"], np.float64).reshape(Cp, H)
        else:
            if B != Q:
                raise ValueError("a normalized-input pair bias needs batch == queries")
            P = Xn
            Wb = np.asarray(pair_bias["projectionWeight"], np.float64).reshape(C, H)
        bias = np.einsum("qkc,ch->hqk", P, Wb)
        logits = logits + bias[None]
    logits = np.clip(logits, -1e8, 1e8)
    logits = logits - logits.max(axis=-1, keepdims=True)
    a = np.exp(logits)
    a /= a.sum(axis=-1, keepdims=True)
    o = np.einsum("bhqk,bkhd->bqhd", a, v) * g
    y = o.reshape(B, Q, C) @ w["outputWeight"].reshape(C, C) + w["outputBias"]
    if transpose:
        y = y.transpose(1, 0, 2)
    return y.reshape(-1).astype(np.float32)
