"""NumPy oracle for the escha coded projection — TEST INFRASTRUCTURE ONLY.

A from-scratch restatement of the contract in escha_mlx/ref.py (the reference's
bit-exact NumPy codec) plus the fixed accumulation order of the reference GPU
GEMV (escha_mlx/msl.py:205-308).  Only tests/, __graft_entry__.smoke() and
bench.py's cpu_baseline leg may import this module.

Pinning status of each function (what checks it independently of its own code):

  cba_lut          pinned: full-table SHA-256 of the hash closed form computed
                   with Python ints (tests/test_oracle.py), and the decode goldens.
  tile_states /    pinned: the reference's committed decode goldens
  reconstruct      (tests/data/codec, copied to tests/golden) bit-for-bit,
                   K=2 (2048x1024) and K=3 (512x2048); brute-force bit-string
                   windows on random tiles.
  lane_map         pinned: bijection + the goldens (a wrong map fails them).
  h128             pinned: Sylvester-matrix closed form (f64) + involution; bit
                   order pinned by vectors written from escha_mlx/ref.py
                   (tests/golden/make_ref_vectors.py).
  input_transform, pinned: vectors written from escha_mlx/ref.py (bit-exact).
  output_transform
  swiglu           pinned: vectors written from escha_mlx/ref.py (bit-exact
                   on this host's libm/numpy exp).
  fold_scales      pinned: known answers (tests/test_dense_linear.py:43-62 of
                   the reference) restated in tests/test_oracle.py.
  gemv_ordered     pinned: f64 exact product (tolerance), row-wise brute force
                   sequential float32 loop on tiny shapes, and one-hot inputs
                   (exact weight read-back).
  expert_linear    pinned: real-data "deploy" corners (tolerance, reference
                   tests/test_dense_linear.py:68-78) + vectors from ref.py
                   (tolerance: numpy BLAS order is host-dependent).
  route_topk       pinned: stable argsort closed form; vectors from ref.py.
  build_groups     pinned: independent brute-force loop model + invariants
                   (tests/test_blocked.py:25-66 of the reference).
  moe_routed       pinned by composition of the above; f64 variant checked
                   against vectors from ref.moe_block's routed sum.
  w8a16            pinned: the reference's w8a16 goldens (tests/data/codec/
                   w8a16_*, tolerance: float32 sum order) and one-hot inputs
                   (each output is one contract weight f16(f32(w8)*f32(scale))).
  q8_dequant,      pinned: exact rational products w8 * scale rounded once to
  q8_embed         f16 (f16 scales: the float32 product is exact), for all 256
                   int8 values, and the one-hot w8a16 check above.
  linear_f16,      pinned: vectors from ref.moe_block with a non-zero shared
  shared_act,      expert and router (tests/golden/make_ref_vectors.py),
  moe_block        tolerance (numpy BLAS order, f64 routed sum).
"""
from __future__ import annotations

import numpy as np

M32 = 0xFFFFFFFF
# 1/sqrt(128) as the exact float32 the format pins (escha_mlx/ref.py:30).
RS = np.float32(0.088388347648)
HASH_MUL = 0xCBAC1FED
HASH_MASK = 0x8FFF8FFF
HASH_XOR = 0x3B603B60


# ---------------------------------------------------------------- codebook

def cba_lut() -> np.ndarray:
    """All 65,536 decoded values, state -> f16 (escha_mlx/ref.py:37-48).

    r = ((s * 0xCBAC1FED) mod 2^32 & 0x8FFF8FFF) ^ 0x3B603B60, value =
    f16(lo16(r)) + f16(hi16(r)) rounded to nearest-even.  The two halves have
    exponent field 011xx, so their exact sum fits a float32 and one cast to
    f16 is the correctly rounded f16 addition.
    """
    s = np.arange(65536, dtype=np.uint64)
    r = ((s * np.uint64(HASH_MUL)) & np.uint64(M32))
    r = (r & np.uint64(HASH_MASK)) ^ np.uint64(HASH_XOR)
    lo = (r & np.uint64(0xFFFF)).astype(np.uint16).view(np.float16).astype(np.float32)
    hi = (r >> np.uint64(16)).astype(np.uint16).view(np.float16).astype(np.float32)
    return (lo + hi).astype(np.float16)


LUT = cba_lut()


# ---------------------------------------------------------------- tile layout

def code_words(code: np.ndarray) -> np.ndarray:
    """int16/uint16 [..., 16K] -> little-endian uint32 words [..., 8K].

    word w = u16[2w] | u16[2w+1] << 16 (escha_mlx/ref.py:58-61,
    escha_mlx/msl.py:1398-1401).  Written with shifts so it holds on any host.
    """
    u = np.ascontiguousarray(code).view(np.uint16).astype(np.uint32)
    return (u[..., 0::2] | (u[..., 1::2] << np.uint32(16))).astype(np.uint32)


def _window_tables(K: int):
    """Per trellis step t: the word holding its window's first bit, and the bit
    offset inside that word.

    The tile's words form one circular bitstream of N = 256K bits, word 0 bit 31
    first.  Step t's 16-bit state is the window of bits [K(t+1)-16, K(t+1))
    (mod N) read MSB-first — the tail-biting trellis of escha_mlx/ref.py:64-93.
    """
    n = 256 * K
    start = (K * (np.arange(256) + 1) - 16) % n
    return start // 32, start % 32


def tile_states(words: np.ndarray, K: int) -> np.ndarray:
    """words [T, 8K] uint32 -> states [T, 256] uint16 (trellis step order)."""
    nw = 8 * K
    a, o = _window_tables(K)
    w = words.astype(np.uint64)
    merged = (w[:, a] << np.uint64(32)) | w[:, (a + 1) % nw]
    return ((merged >> (np.uint64(48) - o.astype(np.uint64))) & np.uint64(0xFFFF)).astype(np.uint16)


def lane_map() -> tuple[np.ndarray, np.ndarray]:
    """Trellis step t = 8*lane + j -> (row, col) inside the 16x16 tile.

    row = 2(lane&3) + (j&1) + 8((j>>1)&1);  col = 2((lane>>3) + 4[j>=4]) +
    ((lane>>2)&1)  (escha_mlx/ref.py:96-111).  row indexes input channels,
    col output channels (y = x @ W).
    """
    t = np.arange(256)
    lane, j = t >> 3, t & 7
    row = 2 * (lane & 3) + (j & 1) + 8 * ((j >> 1) & 1)
    col = 2 * ((lane >> 3) + 4 * (j >= 4)) + ((lane >> 2) & 1)
    return row, col


_ROW, _COL = lane_map()


def reconstruct(code: np.ndarray, ic: int, oc: int, K: int, lut: np.ndarray | None = None,
                chunk_tiles: int = 1 << 16) -> np.ndarray:
    """Packed code [IC/16, OC/16, 16K] (or u32 [.., 8K]) -> bare weight [IC, OC] f16.

    Follows escha_mlx/ref.py:126-134 / 173-197 (tile (kt, nt) holds
    W[16kt:16kt+16, 16nt:16nt+16]).  Processes tiles in chunks so that large
    projections stay within memory.
    """
    lut = LUT if lut is None else lut
    tk, tn = ic // 16, oc // 16
    if code.dtype == np.uint32:
        words = code.reshape(tk * tn, 8 * K)
    else:
        words = code_words(code.reshape(tk * tn, 16 * K))
    out = np.empty((tk * tn, 16, 16), dtype=np.float16)
    for s in range(0, tk * tn, chunk_tiles):
        st = tile_states(words[s:s + chunk_tiles], K)
        vals = lut[st]
        blk = np.empty((vals.shape[0], 16, 16), dtype=np.float16)
        blk[:, _ROW, _COL] = vals
        out[s:s + chunk_tiles] = blk
    return out.reshape(tk, tn, 16, 16).transpose(0, 2, 1, 3).reshape(ic, oc)


def decode_tile(words: np.ndarray, K: int, lut: np.ndarray | None = None) -> np.ndarray:
    """One tile's 8K code words -> its 16x16 f16 block (escha_mlx/ref.py:114-123):
    the tile's 256 trellis states through the value table, placed by the lane
    map."""
    lut = LUT if lut is None else lut
    vals = lut[tile_states(np.asarray(words, dtype=np.uint32).reshape(1, 8 * K), K)[0]]
    tile = np.zeros((16, 16), dtype=np.float16)
    tile[_ROW, _COL] = vals
    return tile


def reconstruct_tiles(code: np.ndarray, ic: int, oc: int, K: int) -> np.ndarray:
    """The reference's literal form of reconstruct: a Python loop over the
    tiles (kt, nt), one decode_tile each (escha_mlx/ref.py:126-134).  Same
    weights as reconstruct; kept as the CPU baseline's un-vectorised timing."""
    tk, tn = ic // 16, oc // 16
    if code.dtype == np.uint32:
        words = code.reshape(tk, tn, 8 * K)
    else:
        words = code_words(code.reshape(tk * tn, 16 * K)).reshape(tk, tn, 8 * K)
    out = np.zeros((ic, oc), dtype=np.float16)
    for kt in range(tk):
        for nt in range(tn):
            out[16 * kt:16 * kt + 16, 16 * nt:16 * nt + 16] = decode_tile(words[kt, nt], K)
    return out


# ---------------------------------------------------------------- transforms

def h128(x: np.ndarray) -> np.ndarray:
    """Unnormalised Sylvester-order WHT on contiguous 128-blocks of the last axis.

    Radix-2 butterfly, stage s pairs i and i^(1<<s) for s = 0..6, (a+b, a-b) in
    float32 (escha_mlx/ref.py:204-218; same stage order as msl.py:905-913).
    """
    n = x.shape[-1]
    if n % 128:
        raise ValueError(f"H128 needs a multiple of 128, got {n}")
    y = np.ascontiguousarray(x, dtype=np.float32).reshape(-1, 128)
    for s in range(7):
        h = 1 << s
        v = y.reshape(-1, 128 // (2 * h), 2, h)
        a, b = v[:, :, 0, :], v[:, :, 1, :]
        y = np.stack([a + b, a - b], axis=2).reshape(-1, 128)
    return y.reshape(x.shape)


def input_transform(x: np.ndarray, rin: np.ndarray) -> np.ndarray:
    """xh = f16(H128(f32(x) * f32(rin)) * RS)  (escha_mlx/ref.py:221-223)."""
    return (h128(x.astype(np.float32) * rin.astype(np.float32)) * RS).astype(np.float16)


def output_transform(mid: np.ndarray, rout: np.ndarray) -> np.ndarray:
    """y = f16((H128(mid) * RS) * rout), two f32 multiplies (escha_mlx/ref.py:226-228)."""
    return ((h128(mid.astype(np.float32)) * RS) * rout.astype(np.float32)).astype(np.float16)


def fold_scales(rin, rout, s_in=None, s_out=None):
    """rin*s_in, rout*s_out as float32 products (escha_mlx/ref.py:242-277)."""
    ri = rin.astype(np.float32)
    ro = rout.astype(np.float32)
    if s_in is not None:
        ri = ri * s_in.astype(np.float32)
    if s_out is not None:
        ro = ro * s_out.astype(np.float32)
    return ri, ro


def swiglu(gu16: np.ndarray) -> np.ndarray:
    """h = f16(f16(g / (1 + exp(-g))) * u), gate = first half (escha_mlx/ref.py:296-301)."""
    i = gu16.shape[-1] // 2
    g = gu16[..., :i].astype(np.float32)
    s16 = (g / (np.float32(1.0) + np.exp(-g))).astype(np.float16)
    return (s16.astype(np.float32) * gu16[..., i:].astype(np.float32)).astype(np.float16)


# ---------------------------------------------------------------- GEMV

def gemv_ordered(xh: np.ndarray, w: np.ndarray) -> np.ndarray:
    """mid = xh @ w in the reference GPU kernels' exact float32 order.

    For output column c and quarter p, a_p starts at +0 and, for kt ascending,
    adds x[16kt+r]*w[16kt+r, c] for r = 2p, 2p+1, 2p+8, 2p+9 in that order; the
    result is (a0 + a1) + (a2 + a3) (escha_mlx/msl.py:205-308, the xor-1 then
    xor-2 shuffle reduction; identical in the staged, row-blocked and fused-out
    kernels, msl.py:389-435, 438-597, 688-872).  f16 x f16 products are exact
    in float32, so fused or unfused multiply-add give the same bits; only the
    order matters and it is reproduced here exactly.

    xh [M, IC] f16, w [IC, OC] f16 -> [M, OC] float32.
    """
    m, ic = xh.shape
    oc = w.shape[1]
    x = xh.astype(np.float32)
    wf = w.astype(np.float32)
    acc = np.zeros((4, m, oc), dtype=np.float32)
    offs = (0, 1, 8, 9)
    for kt in range(ic // 16):
        for off in offs:
            rows = 16 * kt + 2 * np.arange(4) + off            # one row per quarter p
            prod = x[:, rows].T[:, :, None] * wf[rows][:, None, :]  # [4, M, OC], exact
            acc += prod
    return (acc[0] + acc[1]) + (acc[2] + acc[3])


def gemv_f64(xh: np.ndarray, w: np.ndarray) -> np.ndarray:
    """Exact-product reference in float64 (the tolerance anchor)."""
    return xh.astype(np.float64) @ w.astype(np.float64)


def expert_linear(x, code, rin, rout, K, w_bare=None, ordered=False):
    """x [M, IC] -> [M, OC] f16 (escha_mlx/ref.py:231-239).

    ``ordered=False`` multiplies with numpy's float32 matmul as the reference
    does (BLAS summation order, host dependent); ``ordered=True`` uses the GPU
    kernel order of ``gemv_ordered`` so the result is reproducible bit-for-bit.
    """
    ic, oc = rin.shape[-1], rout.shape[-1]
    if w_bare is None:
        w_bare = reconstruct(code, ic, oc, K)
    xh = input_transform(x, rin)
    mid = gemv_ordered(xh, w_bare) if ordered else xh.astype(np.float32) @ w_bare.astype(np.float32)
    return output_transform(mid, rout)


def dense_linear(x, code, rin, rout, K, bias=None, ordered=False):
    """expert_linear plus the optional f16 bias added in f32 (escha_mlx/ref.py:280-293)."""
    y = expert_linear(x, code, rin, rout, K, ordered=ordered)
    if bias is None:
        return y
    return (y.astype(np.float32) + bias.astype(np.float32)).astype(np.float16)


# ---------------------------------------------------------------- routing / MoE

def route_topk(logits: np.ndarray, top_k: int):
    """fp32 logits [T, E] -> (ids [T, k] int32, scores [T, k] f32).

    Stable descending order (ties -> lower expert id first), softmax over the k
    selected values with the max subtracted (escha_mlx/ref.py:326-331).
    """
    lg = logits.astype(np.float32)
    ids = np.argsort(-lg, axis=-1, kind="stable")[:, :top_k]
    top = np.take_along_axis(lg, ids, axis=-1)
    e = np.exp(top - top.max(axis=-1, keepdims=True))
    return ids.astype(np.int32), (e / e.sum(axis=-1, keepdims=True)).astype(np.float32)


def n_groups_bound(m: int, E: int, R: int) -> int:
    """Static bound on R-row groups: every expert may waste R-1 slots (escha_mlx/moe.py:81-83)."""
    return (m + E * (R - 1) + R - 1) // R


def build_groups(row_expert: np.ndarray, E: int, R: int, n_groups: int):
    """Rows sorted (stably) by expert, packed into R-row groups (escha_mlx/moe.py:30-78).

    Returns rows_idx [n_groups*R] (padding slots = m, the caller's zero sink row)
    and group_expert [n_groups] (-1 past the last occupied group).
    """
    m = len(row_expert)
    rows_idx = np.full(n_groups * R, m, dtype=np.int32)
    group_expert = np.full(n_groups, -1, dtype=np.int32)
    slot = 0
    for e in range(E):
        members = [r for r in range(m) if row_expert[r] == e]
        if not members:
            continue
        ng = (len(members) + R - 1) // R
        rows_idx[slot:slot + len(members)] = members
        group_expert[slot // R: slot // R + ng] = e
        slot += ng * R
    return rows_idx, group_expert


def moe_routed(x, ids, scores, gu, dn, K_gu, K_dn, ordered=True, acc64=False):
    """Routed-expert sum for T tokens (models/qwen3_5_moe.py:207-253, ref.py:332-342).

    gu / dn: dicts with 'w' [E, IC, OC] f16 decoded weights (or 'code'),
    'rin' [E, IC] f32, 'rout' [E, OC] f32.  Rows are token-major (slot s of
    token t is row t*k+s).  Per row: gate_up linear -> swiglu -> down linear ->
    d16; contrib = f32(d16) * f32(f16(score)); summed over slots in fixed slot
    order in float32 (the kernel contract) or float64 (``acc64``, as
    ref.moe_block does); the sum is rounded to f16.
    """
    t, k = ids.shape
    out = np.zeros((t, x.shape[1]), dtype=np.float64 if acc64 else np.float32)
    for ti in range(t):
        for s in range(k):
            e = int(ids[ti, s])
            h = expert_linear(x[ti:ti + 1], None, gu["rin"][e], gu["rout"][e], K_gu,
                              w_bare=gu["w"][e], ordered=ordered)
            h = swiglu(h)
            d = expert_linear(h, None, dn["rin"][e], dn["rout"][e], K_dn,
                              w_bare=dn["w"][e], ordered=ordered)
            w16 = np.float32(np.float16(scores[ti, s]))
            c = d[0].astype(np.float32) * w16
            out[ti] = out[ti] + (c.astype(np.float64) if acc64 else c)
    return out.astype(np.float16)


# ---------------------------------------------------------------- dense int8 / full MoE block

def q8_dequant(w8: np.ndarray, scale: np.ndarray) -> np.ndarray:
    """The contract weights wf = f16(f32(w8) * f32(scale)), w8 [N, K] int8,
    scale [N] (escha_mlx/quant.py:1-30, ref.py:308-311)."""
    return (w8.astype(np.float32) * np.asarray(scale, np.float32)[:, None]).astype(np.float16)


def w8a16(x: np.ndarray, w8: np.ndarray, scale: np.ndarray) -> np.ndarray:
    """y = f16(f32(x) @ f32(wf)^T), wf = q8_dequant(w8, scale); w8 [O, K]
    int8, scale [O] (escha_mlx/ref.py:308-311, quant.py:1-30)."""
    wf = q8_dequant(w8, scale)
    return (x.astype(np.float32) @ wf.astype(np.float32).T).astype(np.float16)


def q8_embed(ids: np.ndarray, w8: np.ndarray, scale: np.ndarray) -> np.ndarray:
    """Embedding rows q8_dequant(w8, scale)[ids] (escha_mlx/quant.py:253-266:
    the affine dequant there is exact in float32, then one f16 rounding)."""
    ids = np.asarray(ids)
    rows = q8_dequant(w8[ids.reshape(-1)], np.asarray(scale)[ids.reshape(-1)])
    return rows.reshape(*ids.shape, w8.shape[1])


def linear_f16(x: np.ndarray, w: np.ndarray) -> np.ndarray:
    """A bias-free f16 Linear: f16(f32(x) @ f32(w)^T) (the router and shared
    gates, escha_mlx/ref.py:324, 347)."""
    return (x.astype(np.float32) @ w.astype(np.float32).T).astype(np.float16)


def shared_act(g16: np.ndarray, u16: np.ndarray) -> np.ndarray:
    """f16((g / (1 + exp(-g))) * u) in float32 (escha_mlx/ref.py:345)."""
    g = g16.astype(np.float32)
    return ((g / (np.float32(1.0) + np.exp(-g))) * u16.astype(np.float32)).astype(np.float16)


def moe_block(x, w, top_k, ids=None, scores=None, K_gu=2, K_dn=3, routed_f16=True):
    """Full MoE block (escha_mlx/ref.py:314-349; models/qwen3_5_moe.py:257-273).

    w: gate_w [E, H] f16; gu / dn dicts as in moe_routed; sh_{gate,up,down}_w8 /
    _scale; shg_w [1, H] f16.  Router: f16-rounded logits, top-k (stable),
    softmax over the k values; ids/scores may be injected.  routed_f16 rounds
    the routed sum to f16 before the shared expert is added (the model's
    forward contract, models/qwen3_5_moe.py:250-253); False keeps
    ref.moe_block's float64 routed sum.
    """
    logits = linear_f16(x, w["gate_w"]).astype(np.float32)
    if ids is None:
        ids, scores = route_topk(logits, top_k)
    if routed_f16:
        y = moe_routed(x, ids, scores, w["gu"], w["dn"], K_gu, K_dn, ordered=False).astype(np.float32)
    else:
        y = _routed_f64(x, ids, scores, w["gu"], w["dn"], K_gu, K_dn)
    g = w8a16(x, w["sh_gate_w8"], w["sh_gate_scale"])
    u = w8a16(x, w["sh_up_w8"], w["sh_up_scale"])
    hh = shared_act(g, u)
    sh = w8a16(hh, w["sh_down_w8"], w["sh_down_scale"]).astype(np.float32)
    shg = linear_f16(x, w["shg_w"]).astype(np.float32)
    sgate = np.float32(1.0) / (np.float32(1.0) + np.exp(-shg))
    return (y + sh * sgate).astype(np.float16)


def _routed_f64(x, ids, scores, gu, dn, K_gu, K_dn):
    t, k = ids.shape
    out = np.zeros((t, x.shape[1]), dtype=np.float64)
    for ti in range(t):
        for s in range(k):
            e = int(ids[ti, s])
            h = expert_linear(x[ti:ti + 1], None, gu["rin"][e], gu["rout"][e], K_gu,
                              w_bare=gu["w"][e])
            h = swiglu(h)
            d = expert_linear(h, None, dn["rin"][e], dn["rout"][e], K_dn, w_bare=dn["w"][e])
            out[ti] += (d[0].astype(np.float32) * np.float32(np.float16(scores[ti, s]))).astype(np.float64)
    return out
