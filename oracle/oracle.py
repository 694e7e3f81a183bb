"""CPU oracle of the routed-expert MoE hot path -- TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg import
this module, as the checker (or the timed CPU baseline).  The product package
never imports it.

It restates the reference's PyTorch algorithm with numpy and the C routines of
hsmoe_oracle.c (liboracle.so); each function names the reference lines it
follows.  bf16 tensors are numpy uint16 arrays of raw bf16 bits.

Parity pins (tests/test_oracle_*.py): the reference's own KATs (stable top-k,
E8M0 127/128/126, dequant interleave / per-group scale, SiLU-not-sigmoid,
scaling-factor sum, MTP accept/reject cases), torch's own casts for every
format conversion, torch's own bf16 ops running the reference's FFN and
router formulas on inputs whose sums are exact, float64 evaluations,
splitmix64's published outputs, and brute-force / closed forms on small
inputs.  Every function is pinned by at least one of them.
"""
from __future__ import annotations

import ctypes
from pathlib import Path

import numpy as np

_HERE = Path(__file__).resolve().parent
_LIB_PATH = _HERE / "_build" / "liboracle.so"
_lib = None

MASK64 = (1 << 64) - 1


def lib():
    global _lib
    if _lib is None:
        if not _LIB_PATH.exists():
            from oracle.build import build_oracle
            build_oracle()
        L = ctypes.CDLL(str(_LIB_PATH))
        P = ctypes.c_void_p
        i64, u64, f32, i32 = ctypes.c_int64, ctypes.c_uint64, ctypes.c_float, ctypes.c_int
        sig = {
            "hso_bf16_to_f32": (f32, [ctypes.c_uint16]),
            "hso_f32_to_bf16": (ctypes.c_uint16, [f32]),
            "hso_f64_to_bf16": (ctypes.c_uint16, [ctypes.c_double]),
            "hso_e2m1": (f32, [i32]),
            "hso_e8m0_cast": (f32, [ctypes.c_uint8]),
            "hso_e8m0_shift": (f32, [ctypes.c_uint8]),
            "hso_e4m3": (f32, [ctypes.c_uint8]),
            "hso_dequant_fp4": (None, [P, P, i64, i64, P]),
            "hso_dequant_fp8_block": (None, [P, P, i64, i64, P]),
            "hso_logits_bf16": (None, [P, P, P, i64, i64, i64, P]),
            "hso_rand": (u64, [u64, u64]),
            "hso_key": (u64, [u64, u64]),
            "hso_gen_bytes": (None, [u64, i64, P]),
            "hso_gen_e4m3": (None, [u64, i64, P]),
            "hso_gen_e8m0": (None, [u64, i64, i32, i32, P]),
            "hso_gen_normal_f32": (None, [u64, i64, f32, f32, P]),
            "hso_gen_normal_bf16": (None, [u64, i64, f32, f32, P]),
            "hso_gen_uniform_f32": (None, [u64, i64, f32, f32, f32, P]),
            "hso_gen_index": (None, [u64, i64, i64, P]),
        }
        for name, (res, args) in sig.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def _p(a: np.ndarray):
    assert a.flags["C_CONTIGUOUS"]
    return a.ctypes.data_as(ctypes.c_void_p)


# ------------------------------------------------------------------ formats

def bf16_to_f32(h: np.ndarray) -> np.ndarray:
    return (np.asarray(h, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def f32_to_bf16(f: np.ndarray) -> np.ndarray:
    """Round to nearest even, NaN -> 0x7FC0 (torch's .to(torch.bfloat16))."""
    u = np.ascontiguousarray(f, dtype=np.float32).view(np.uint32)
    r = ((u + np.uint32(0x7FFF) + ((u >> 16) & np.uint32(1))) >> 16).astype(np.uint16)
    r[(u & np.uint32(0x7FFFFFFF)) > np.uint32(0x7F800000)] = 0x7FC0
    return r


def to_np_bf16(t) -> np.ndarray:
    """torch bf16 tensor (any device) -> numpy uint16 bits."""
    import torch
    return t.detach().contiguous().view(torch.int16).cpu().numpy().view(np.uint16)


E2M1 = None


def e2m1_table() -> np.ndarray:
    """The 16 e2m1 values (_fp4.py:79-90, fused_moe.py:604-608)."""
    global E2M1
    if E2M1 is None:
        E2M1 = np.array([lib().hso_e2m1(c) for c in range(16)], dtype=np.float32)
    return E2M1


def e8m0_table(semantics: str = "cast") -> np.ndarray:
    """256 fp32 scale values: "cast" = torch float8_e8m0fnu -> float32 (engine.py:1260-1271);
    "shift" = bits e << 23 (weight_loader.py:14-19)."""
    fn = lib().hso_e8m0_cast if semantics == "cast" else lib().hso_e8m0_shift
    return np.array([fn(e) for e in range(256)], dtype=np.float32)


def e4m3_table() -> np.ndarray:
    return np.array([lib().hso_e4m3(b) for b in range(256)], dtype=np.float32)


# ------------------------------------------------------------------ dequant

def dequant_fp4(packed: np.ndarray, scale: np.ndarray, e8m0: bool = True, semantics: str = "cast") -> np.ndarray:
    """bf16 [N, K] from packed [N, K/2] + scales [N, K/32] (fused_moe.py:22-26; weight_loader.py:35-45).
    e8m0=True: scale holds E8M0 bytes; else fp32 scale values."""
    packed = np.ascontiguousarray(packed).view(np.uint8)
    n, kh = packed.shape
    k = kh * 2
    if e8m0:
        sf = e8m0_table(semantics)[np.asarray(scale).view(np.uint8)]
    else:
        sf = np.asarray(scale, dtype=np.float32)
    sf = np.ascontiguousarray(np.broadcast_to(sf, (n, k // 32)), dtype=np.float32)
    out = np.empty((n, k), dtype=np.uint16)
    lib().hso_dequant_fp4(_p(packed), _p(sf), n, k, _p(out))
    return out


def dequant_fp8(data: np.ndarray, scale: np.ndarray) -> np.ndarray:
    """bf16 [N, K] from e4m3 [N, K] and fp32 [N/128, K/128] (cast_back, _fp4.py:98-110)."""
    data = np.ascontiguousarray(data).view(np.uint8)
    n, k = data.shape
    sf = np.ascontiguousarray(scale, dtype=np.float32)
    out = np.empty((n, k), dtype=np.uint16)
    lib().hso_dequant_fp8_block(_p(data), _p(sf), n, k, _p(out))
    return out


def cast_back(data: np.ndarray, fp4: bool, scale: np.ndarray, block: tuple[int, int], out_f32: bool) -> np.ndarray:
    """_fp4.py:98-110 for any block: the decoded values (unpack_from_e2m1fn_x2,
    _fp4.py:72-95, or e4m3 -> fp32) times the scale of each element's
    (block[0] x block[1]) block -- the scales repeat_interleave'd along both
    axes and cut to the data's shape -- as one fp32 multiply; returned as fp32,
    or as bf16 bits (RNE).  data: packed FP4 bytes [N, K/2] or e4m3 bytes [N, K]."""
    data = np.ascontiguousarray(data).view(np.uint8)
    if fp4:
        codes = np.empty((data.shape[0], data.shape[1] * 2), dtype=np.uint8)
        codes[:, 0::2] = data & 0x0F
        codes[:, 1::2] = data >> 4
        vals = e2m1_table()[codes]
    else:
        vals = e4m3_table()[data]
    n, k = vals.shape
    sf = np.asarray(scale, dtype=np.float32)
    sf = np.repeat(np.repeat(sf, block[0], axis=0), block[1], axis=1)[:n, :k]
    prod = (vals.astype(np.float32) * sf).astype(np.float32)
    return prod if out_f32 else f32_to_bf16(prod)


def xor_checksum(buf: np.ndarray) -> np.ndarray:
    """uint8 [16]: the XOR of the buffer's 16-byte words (hsmoe_xor_checksum;
    no reference counterpart: the store-integrity check of this build)."""
    b = np.ascontiguousarray(buf).view(np.uint8).reshape(-1)
    if b.size % 16:
        raise ValueError("xor_checksum takes a multiple of 16 bytes")
    if b.size == 0:
        return np.zeros(16, dtype=np.uint8)
    return np.bitwise_xor.reduce(b.view(np.uint64).reshape(-1, 2), axis=0).view(np.uint8)


# ------------------------------------------------------------------ RNG (workload generator)

KIND_FP4_DATA, KIND_FP4_SCALE, KIND_GATE_W, KIND_GATE_BIAS, KIND_HIDDEN = 1, 2, 3, 4, 5
KIND_SHARED_DATA, KIND_SHARED_SCALE, KIND_LM_HEAD, KIND_NORM_W, KIND_RESIDUAL = 6, 7, 8, 9, 10
KIND_DRAFT, KIND_TID2EID = 11, 12


def tag(kind: int, layer: int = 0, eid: int = 0, sub: int = 0) -> int:
    kind, layer, eid, sub = int(kind), int(layer), int(eid), int(sub)
    return ((kind & 0xFF) << 56) | ((layer & 0xFFFF) << 40) | ((eid & 0xFFFFFFFF) << 8) | (sub & 0xFF)


def key(seed: int, t: int) -> int:
    return lib().hso_key(int(seed) & MASK64, int(t) & MASK64)


def gen_bytes(k: int, n: int) -> np.ndarray:
    out = np.empty(n, dtype=np.uint8)
    lib().hso_gen_bytes(k, n, _p(out))
    return out


def gen_e4m3(k: int, n: int) -> np.ndarray:
    out = np.empty(n, dtype=np.uint8)
    lib().hso_gen_e4m3(k, n, _p(out))
    return out


def gen_e8m0(k: int, n: int, lo: int = 119, span: int = 6) -> np.ndarray:
    out = np.empty(n, dtype=np.uint8)
    lib().hso_gen_e8m0(k, n, lo, span, _p(out))
    return out


def gen_normal_bf16(k: int, n: int, mean: float, std: float) -> np.ndarray:
    out = np.empty(n, dtype=np.uint16)
    lib().hso_gen_normal_bf16(k, n, mean, std, _p(out))
    return out


def gen_normal_f32(k: int, n: int, mean: float, std: float) -> np.ndarray:
    out = np.empty(n, dtype=np.float32)
    lib().hso_gen_normal_f32(k, n, mean, std, _p(out))
    return out


def gen_uniform_f32(k: int, n: int, lo: float, hi: float, mul: float = 1.0) -> np.ndarray:
    out = np.empty(n, dtype=np.float32)
    lib().hso_gen_uniform_f32(k, n, lo, hi, mul, _p(out))
    return out


def gen_index(k: int, n: int, n_values: int) -> np.ndarray:
    out = np.empty(n, dtype=np.int64)
    lib().hso_gen_index(k, n, n_values, _p(out))
    return out


def gen_fp4_expert(seed: int, layer: int, eid: int, d: int, i: int) -> dict:
    """Raw FP4 expert (packed uint8 + E8M0 bytes) and its bf16 dequantisation."""
    ex = {}
    for sub, (name, rows, cols) in enumerate((("w1", i, d), ("w3", i, d), ("w2", d, i))):
        p = gen_bytes(key(seed, tag(KIND_FP4_DATA, layer, eid, sub)), rows * cols // 2).reshape(rows, cols // 2)
        s = gen_e8m0(key(seed, tag(KIND_FP4_SCALE, layer, eid, sub)), rows * cols // 32).reshape(rows, cols // 32)
        ex[name] = p
        ex[name + "_scale"] = s
        ex[name + "_bf16"] = dequant_fp4(p, s, e8m0=True)
    return ex


def gen_shared_expert(seed: int, layer: int, d: int, i: int) -> dict:
    """FP8 e4m3 shared expert with fp32 128x128 block scales U(0.5, 2)/448, and its bf16 dequantisation."""
    ex = {}
    for sub, (name, rows, cols) in enumerate((("w1", i, d), ("w3", i, d), ("w2", d, i))):
        q = gen_e4m3(key(seed, tag(KIND_SHARED_DATA, layer, 0, sub)), rows * cols).reshape(rows, cols)
        s = gen_uniform_f32(key(seed, tag(KIND_SHARED_SCALE, layer, 0, sub)), (rows // 128) * (cols // 128),
                            0.5, 2.0, np.float32(1.0 / 448.0)).reshape(rows // 128, cols // 128)
        ex[name] = q
        ex[name + "_scale"] = s
        ex[name + "_bf16"] = dequant_fp8(q, s)
    return ex


# ------------------------------------------------------------------ router

def logits_bf16(x: np.ndarray, w: np.ndarray, bias: np.ndarray | None = None) -> np.ndarray:
    """bf16(x . w^T) with the exact sum rounded once; with bias: bf16(logit + bf16(bias)) (router.py:27-29)."""
    x = np.ascontiguousarray(x, dtype=np.uint16)
    w = np.ascontiguousarray(w, dtype=np.uint16)
    m, d = x.shape
    n = w.shape[0]
    out = np.empty((m, n), dtype=np.uint16)
    b = None if bias is None else np.ascontiguousarray(bias, dtype=np.float32)
    lib().hso_logits_bf16(_p(x), _p(w), None if b is None else _p(b), m, n, d, _p(out))
    return out


def softplus_f32(x: np.ndarray) -> np.ndarray:
    """F.softplus (beta 1, threshold 20) in fp32."""
    x = x.astype(np.float32)
    with np.errstate(over="ignore"):
        return np.where(x > np.float32(20.0), x, np.log1p(np.exp(x)).astype(np.float32)).astype(np.float32)


def stable_topk(scores: np.ndarray, k: int) -> np.ndarray:
    """router.py:5-7: descending, ties keep the lower index (stable sort)."""
    order = np.argsort(-scores, axis=1, kind="stable")
    return order[:, :k].astype(np.int64)


def router(x: np.ndarray, gate: np.ndarray, bias: np.ndarray | None, top_k: int = 6, scaling: float = 1.5,
           return_scores: bool = False):
    """compute_expert_affinity_with_bias (router.py:22-36) -> (idx int64 [M, k], w fp32 [M, k])."""
    lg = logits_bf16(x, gate, bias)
    scores = np.sqrt(softplus_f32(bf16_to_f32(lg))).astype(np.float32)
    idx = stable_topk(scores, top_k)
    raw = np.take_along_axis(scores, idx, axis=1)
    s = np.zeros(raw.shape[0], dtype=np.float32)
    for j in range(top_k):
        s = (s + raw[:, j]).astype(np.float32)
    s = np.maximum(s, np.float32(1e-20))
    w = ((raw / s[:, None]).astype(np.float32) * np.float32(scaling)).astype(np.float32)
    if return_scores:
        return idx, w, scores, lg
    return idx, w


# ------------------------------------------------------------------ FFN

def _swiglu_f32(g: np.ndarray, u: np.ndarray, limit: float) -> np.ndarray:
    """fused_moe.py:390-394: gate clamped above only, up clamped both sides; SiLU(g) * u in fp32."""
    L = np.float32(limit)
    g = np.where(g > L, L, g).astype(np.float32)
    u = np.where(u < -L, -L, np.where(u > L, L, u)).astype(np.float32)
    with np.errstate(over="ignore"):
        sig = (np.float32(1.0) / (np.float32(1.0) + np.exp(-g))).astype(np.float32)
    return ((g * sig).astype(np.float32) * u).astype(np.float32)


def expert_ffn_fp32(x: np.ndarray, w1: np.ndarray, w3: np.ndarray, w2: np.ndarray, limit: float = 10.0) -> np.ndarray:
    """fused_expert_ffn_pt (fused_moe.py:383-395) with fp32 accumulation and fp32 intermediates -> fp32 [M, D]."""
    return _ffn_f32w(bf16_to_f32(x), bf16_to_f32(w1), bf16_to_f32(w3), bf16_to_f32(w2), limit)


def _ffn_f32w(xf: np.ndarray, w1f: np.ndarray, w3f: np.ndarray, w2f: np.ndarray, limit: float) -> np.ndarray:
    """expert_ffn_fp32 on fp32 copies of x and the weights (the same operations)."""
    gate = xf @ w1f.T
    up = xf @ w3f.T
    act = _swiglu_f32(gate.astype(np.float32), up.astype(np.float32), limit)
    return (act @ w2f.T).astype(np.float32)


def expert_ffn_ref_bf16(x: np.ndarray, w1: np.ndarray, w3: np.ndarray, w2: np.ndarray,
                        limit: float = 10.0, steps: bool = False):
    """fused_expert_ffn_pt (fused_moe.py:383-395) with the reference's bf16
    rounding points: gate/up bf16 (`hidden @ w1.t()`), activation bf16
    (`.to(w1.dtype)`), fp32-accumulated down -> fp32 before the final bf16 store.
    steps=True -> dict of the bf16 bits of gate, up, act and the fp32 out.
    Pinned by torch's own bf16 ops on inputs whose gate/up sums are exact:
    gate/up bit-exact, act and out within one bf16 step."""
    xf = bf16_to_f32(x)
    gate = f32_to_bf16(xf @ bf16_to_f32(w1).T)
    up = f32_to_bf16(xf @ bf16_to_f32(w3).T)
    act = f32_to_bf16(_swiglu_f32(bf16_to_f32(gate), bf16_to_f32(up), limit))
    out = (bf16_to_f32(act) @ bf16_to_f32(w2).T).astype(np.float32)
    return {"gate": gate, "up": up, "act": act, "out": out} if steps else out


def moe_layer_fp32(x: np.ndarray, idx: np.ndarray, w: np.ndarray, experts: dict, shared: dict | None,
                   limit: float = 10.0) -> np.ndarray:
    """Routed + shared FFN (fused_moe.py:458-551, engine.py:1530-1536) in fp32:
    out[m] = sum_j w[m, j] * FFN_{idx[m, j]}(x[m]) + FFN_shared(x[m]).  Ids < 0 or
    missing from `experts` are skipped."""
    m, d = x.shape
    out = np.zeros((m, d), dtype=np.float32)
    for t in range(m):
        for j in range(idx.shape[1]):
            e = int(idx[t, j])
            if e < 0 or e not in experts:
                continue
            ex = experts[e]
            y = expert_ffn_fp32(x[t:t + 1], ex["w1_bf16"], ex["w3_bf16"], ex["w2_bf16"], limit)[0]
            out[t] = (out[t] + np.float32(w[t, j]) * y).astype(np.float32)
    if shared is not None:
        out = (out + expert_ffn_fp32(x, shared["w1_bf16"], shared["w3_bf16"], shared["w2_bf16"], limit)).astype(
            np.float32)
    return out


def moe_layer_fp32_lazy(x: np.ndarray, idx: np.ndarray, w: np.ndarray, expert_fn, shared_fn, limit: float = 10.0,
                        pool=None) -> np.ndarray:
    """moe_layer_fp32 with experts produced on demand by expert_fn(e) (a dict as
    gen_fp4_expert, or None when absent) and the shared one by shared_fn() (or
    None), never held all at once: each distinct expert is generated, its
    weights widened to fp32 once, and its FFN evaluated for every (token, slot)
    that selects it -- each token row alone, with the same operations as
    moe_layer_fp32 -- on `pool` (a concurrent.futures executor) when given.
    The terms are then added in moe_layer_fp32's order, so the result is the
    same bit for bit."""
    m, d = x.shape
    xf = bf16_to_f32(x)
    uses: dict[int, list[int]] = {}
    for t in range(m):
        for j in range(idx.shape[1]):
            e = int(idx[t, j])
            if e >= 0:
                uses.setdefault(e, [])
                if t not in uses[e]:
                    uses[e].append(t)

    def one(e):
        ex = expert_fn(e)
        if ex is None:
            return e, None
        w1f, w3f, w2f = (bf16_to_f32(ex[k]) for k in ("w1_bf16", "w3_bf16", "w2_bf16"))
        return e, {t: _ffn_f32w(xf[t:t + 1], w1f, w3f, w2f, limit)[0] for t in uses[e]}

    def shared_one():
        sh = shared_fn() if shared_fn is not None else None
        if sh is None:
            return None
        return _ffn_f32w(xf, *(bf16_to_f32(sh[k]) for k in ("w1_bf16", "w3_bf16", "w2_bf16")), limit)

    if pool is None:
        ys = dict(one(e) for e in uses)
        ysh = shared_one()
    else:
        fsh = pool.submit(shared_one)
        ys = dict(pool.map(one, list(uses)))
        ysh = fsh.result()
    out = np.zeros((m, d), dtype=np.float32)
    for t in range(m):
        for j in range(idx.shape[1]):
            e = int(idx[t, j])
            if e < 0 or ys.get(e) is None:
                continue
            out[t] = (out[t] + np.float32(w[t, j]) * ys[e][t]).astype(np.float32)
    if ysh is not None:
        out = (out + ysh).astype(np.float32)
    return out


def moe_layer_reference(x: np.ndarray, idx: np.ndarray, w: np.ndarray, experts: dict, shared: dict | None,
                        limit: float = 10.0, steps: bool = False):
    """The reference's T>1 union route (_forward_legacy torch branch, fused_moe.py:458-551)
    plus the bf16 shared add (engine.py:1530-1536), with all its bf16 roundings:
    bf16 gate/up, bf16 activation, bf16 routing weights, bf16 act*ew product,
    fp32-accumulated down over the union, bf16 output; returns bf16 bits
    (steps=True -> dict with the bf16 routing weights "ew" [m, n_union], the
    union "union", the routed sum "routed", the shared output "shared" and "out").
    Pinned by torch's own ops on exact-sum inputs: ew bit-exact, routed and
    out within one bf16 step, the shared add bit-exact."""
    m, d = x.shape
    union = sorted({int(e) for e in idx.reshape(-1) if int(e) >= 0 and int(e) in experts})
    xf = bf16_to_f32(x)
    acc = np.zeros((m, d), dtype=np.float32)
    ew = np.zeros((m, len(union)), dtype=np.float32)
    pos = {e: q for q, e in enumerate(union)}
    for t in range(m):
        for j in range(idx.shape[1]):
            e = int(idx[t, j])
            if e in pos:
                ew[t, pos[e]] = bf16_to_f32(f32_to_bf16(np.float32(w[t, j]).reshape(1)))[0]
    for q, e in enumerate(union):
        ex = experts[e]
        gate = bf16_to_f32(f32_to_bf16(xf @ bf16_to_f32(ex["w1_bf16"]).T))
        up = bf16_to_f32(f32_to_bf16(xf @ bf16_to_f32(ex["w3_bf16"]).T))
        act = bf16_to_f32(f32_to_bf16(_swiglu_f32(gate, up, limit)))
        weighted = bf16_to_f32(f32_to_bf16((act * ew[:, q:q + 1]).astype(np.float32)))
        acc = (acc + weighted @ bf16_to_f32(ex["w2_bf16"]).T).astype(np.float32)
    routed = f32_to_bf16(acc)
    sh, out = None, routed
    if shared is not None:
        sh = f32_to_bf16(expert_ffn_ref_bf16(x, shared["w1_bf16"], shared["w3_bf16"], shared["w2_bf16"], limit))
        out = bf16_add_bits(routed, sh)
    if steps:
        return {"ew": f32_to_bf16(ew), "union": union, "routed": routed, "shared": sh, "out": out}
    return out


def bf16_add_bits(a: np.ndarray, b: np.ndarray) -> np.ndarray:
    """torch's bf16 + bf16: the two values added in fp32, the sum rounded to bf16."""
    return f32_to_bf16((bf16_to_f32(a) + bf16_to_f32(b)).astype(np.float32))


def rms_norm(x: np.ndarray, w: np.ndarray, eps: float = 1e-6) -> np.ndarray:
    """utils.py:6-9: fp32 mean of squares, x * rsqrt(var + eps) * w, back to bf16."""
    xf = bf16_to_f32(x)
    var = np.mean((xf * xf).astype(np.float32), axis=-1, keepdims=True, dtype=np.float32)
    inv = (np.float32(1.0) / np.sqrt((var + np.float32(eps)).astype(np.float32))).astype(np.float32)
    return f32_to_bf16((bf16_to_f32(w) * (xf * inv).astype(np.float32)).astype(np.float32))


# ------------------------------------------------------------------ MTP acceptance

def argmax_first(row_bf16: np.ndarray) -> int:
    """torch.argmax on a bf16 row: first maximal index; NaN counts as the maximum."""
    v = bf16_to_f32(row_bf16)
    nan = np.isnan(v)
    if nan.any():
        return int(np.argmax(nan))
    return int(np.argmax(v))


def mtp_accept(logits: np.ndarray, combined_ids) -> tuple[int, int]:
    """engine.py:2487-2497: walk positions; accept combined[i+1] while argmax(logits[i])
    equals it; the bonus row is the first mismatch, or the last row. -> (n_accept, bonus_row)."""
    t_total = logits.shape[0]
    n = 0
    for i in range(t_total):
        pred = argmax_first(logits[i])
        if i == t_total - 1:
            return n, i
        if pred == int(combined_ids[i + 1]):
            n += 1
        else:
            return n, i
    return n, t_total - 1
