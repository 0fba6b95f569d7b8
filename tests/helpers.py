"""Test helpers: seeded data in the reference's formats and the parity metrics the tests use."""
from __future__ import annotations

import math

import numpy as np

# e4m3fn magnitudes of codes 0..0x7e (0x7f is NaN), exact in f64
_MAG = np.array([(m / 8.0) * 2.0 ** -6 if e == 0 else (1 + m / 8.0) * 2.0 ** (e - 7)
                 for e in range(16) for m in range(8)][:0x7F])


def decode_table() -> np.ndarray:
    t = np.concatenate([_MAG, [np.nan], -_MAG, [np.nan]])
    return t


def encode_e4m3(values: np.ndarray) -> np.ndarray:
    """Nearest e4m3fn code with ties to the even code, saturating at +-448 (table search in f64)."""
    v = np.asarray(values, np.float64)
    a = np.minimum(np.abs(v), 448.0)
    hi = np.clip(np.searchsorted(_MAG, a), 1, len(_MAG) - 1)
    lo = hi - 1
    dlo, dhi = a - _MAG[lo], _MAG[hi] - a
    pick = np.where(dlo < dhi, lo, np.where(dhi < dlo, hi, np.where(lo % 2 == 0, lo, hi)))
    return (pick | np.where(np.signbit(v), 0x80, 0)).astype(np.uint8)


def log_uniform_scales(rng, rows: int, cols: int) -> np.ndarray:
    """[ceil(rows/128), cols/128] scales, log-uniform in [2^-10, 2^-6]."""
    return (2.0 ** rng.uniform(-10, -6, size=((rows + 127) // 128, cols // 128))).astype(np.float32)


def fp8_weight(rng, rows: int, cols: int, scales: np.ndarray) -> np.ndarray:
    """N(0,1) / block scale quantised to e4m3 with saturation."""
    z = rng.standard_normal((rows, cols))
    s = np.repeat(np.repeat(scales.astype(np.float64), 128, 0)[:rows], 128, 1)
    return encode_e4m3(z / s)


def bf16_round(x: np.ndarray) -> np.ndarray:
    """f32 -> bf16 RNE, widened back to f32 (finite inputs)."""
    b = np.asarray(x, np.float32).view(np.uint32).astype(np.uint64)
    r = ((b + 0x7FFF + ((b >> 16) & 1)) & 0xFFFF0000).astype(np.uint32)
    return r.view(np.float32)


def bf16_normal(rng, shape, std=1.0) -> np.ndarray:
    return bf16_round((rng.standard_normal(shape) * std).astype(np.float32))


def to_bf16_bits(x: np.ndarray) -> np.ndarray:
    return (bf16_round(x).view(np.uint32) >> 16).astype(np.uint16)


def from_bf16_bits(b: np.ndarray) -> np.ndarray:
    return (np.asarray(b, np.uint16).astype(np.uint32) << 16).view(np.float32)


def normwise(got: np.ndarray, ref: np.ndarray) -> float:
    """max |got - ref| / max |ref| — the parity metric for f32 accumulation-order differences."""
    return float(np.max(np.abs(got.astype(np.float64) - ref)) / max(np.max(np.abs(ref)), 1e-30))


def rel_l2(got: np.ndarray, ref: np.ndarray) -> float:
    return float(np.linalg.norm(got.astype(np.float64) - ref) / max(np.linalg.norm(ref.astype(np.float64)), 1e-30))


def bf16_ulp(x: np.ndarray) -> np.ndarray:
    a = np.abs(np.asarray(x, np.float64))
    e = np.floor(np.log2(np.maximum(a, 2.0 ** -126)))
    return 2.0 ** (e - 7)


def dequant(w: np.ndarray, s: np.ndarray) -> np.ndarray:
    """Dequantised f64 weight dec(W) * S[r/128, c/128]."""
    rows, cols = w.shape
    return decode_table()[w] * np.repeat(np.repeat(s.astype(np.float64), 128, 0)[:rows], 128, 1)


def condition(w: np.ndarray, s: np.ndarray, x: np.ndarray) -> np.ndarray:
    """sum_c |W[r, c] x[p, c]| per output [rows, n]: the scale of f32 reordering error."""
    return np.abs(np.asarray(x, np.float64)) @ np.abs(dequant(w, s)).T


def within_bf16_cond(got: np.ndarray, ref_bf16: np.ndarray, cond: np.ndarray, rel: float = 1e-5) -> bool:
    """bf16 outputs agree up to one rounding step plus an f32 summation-order error bounded by
    rel * sum|terms| (element-wise relative error is ill-conditioned where terms cancel)."""
    d = np.abs(got.astype(np.float64) - ref_bf16.astype(np.float64))
    bound = bf16_ulp(np.maximum(np.abs(got), np.abs(ref_bf16))) * 1.0000001 + rel * cond
    return bool(np.all(d <= bound))


def within_one_bf16_ulp(got: np.ndarray, ref: np.ndarray) -> bool:
    """bf16 outputs differ from the reference's bf16 outputs by at most one rounding step."""
    d = np.abs(got.astype(np.float64) - ref.astype(np.float64))
    return bool(np.all(d <= bf16_ulp(np.maximum(np.abs(got), np.abs(ref))) * 1.0000001))


def write_safetensors(path, tensors, metadata=None, header_pad=True, raw_header=None):
    """Writes a safetensors file: tensors maps name -> (dtype string, shape, bytes), payloads packed in
    the given order. raw_header replaces the JSON header text (for malformed-file tests)."""
    import json
    import struct
    header, payload, off = {}, b"", 0
    if metadata is not None:
        header["__metadata__"] = metadata
    for name, (dtype, shape, data) in tensors.items():
        header[name] = {"dtype": dtype, "shape": list(shape), "data_offsets": [off, off + len(data)]}
        payload += data
        off += len(data)
    text = raw_header if raw_header is not None else json.dumps(header, separators=(",", ":"))
    hb = text.encode()
    if header_pad:
        hb += b" " * ((-len(hb)) % 8)
    with open(path, "wb") as f:
        f.write(struct.pack("<Q", len(hb)) + hb + payload)
    return path


# ------------------------------------------------------------------ closed-form mode-B layers
def _unit_codes(rng, shape, p_zero):
    """e4m3 codes of magnitude in [1, 2) (0x38..0x3f) with random signs; zero with probability p_zero."""
    c = (0x38 + rng.integers(0, 8, shape)).astype(np.uint8)
    c |= np.where(rng.random(shape) < 0.5, 0x80, 0).astype(np.uint8)
    c[rng.random(shape) < p_zero] = 0
    return c


def _lowbits_chunk(t: np.ndarray) -> np.ndarray:
    b = np.abs(t).view(np.uint64)
    e = (b >> np.uint64(52)).astype(np.int64)                    # biased exponent (0: subnormal or zero)
    mant = b & np.uint64((1 << 52) - 1)
    mant = np.where(e > 0, mant | np.uint64(1 << 52), mant)      # with the implicit bit of normal values
    lb = (mant & (~mant + np.uint64(1))).astype(np.float64)      # its lowest set bit, a power of two < 2^53
    k = (lb.view(np.uint64) >> np.uint64(52)).astype(np.int64) - 1023 + np.maximum(e, 1) - 1075
    normal = ((np.clip(k, -1022, 1023) + 1023).astype(np.uint64) << np.uint64(52)).view(np.float64)
    out = np.where(k >= -1022, normal, np.ldexp(1.0, np.maximum(k, -1074)))
    return np.where(b == 0, 0.0, out)


def _lowbits(t: np.ndarray) -> np.ndarray:
    """The lowest set bit (a power of two) of each dyadic value of t, exact in f64; 0 where t == 0.
    From the f64 bit fields (lowest set bit of the significand, shifted by the exponent), in chunks
    of 2^20 values so the temporaries stay small."""
    t = np.asarray(t, np.float64)
    flat = np.ascontiguousarray(t).reshape(-1)
    out = np.empty_like(flat)
    step = 1 << 20
    for i in range(0, flat.size, step):
        out[i:i + step] = _lowbits_chunk(flat[i:i + step])
    return out.reshape(t.shape)


def exact_in_f32(x: np.ndarray, w: np.ndarray) -> bool:
    """Every partial sum of every x[p] . w[o] (f64 dyadic values), in any order, is exact in f32:
    all products are multiples of q = (lowest bit of x) (lowest bit of w) and sum |x w| < 2^24 q."""
    lx, lw = _lowbits(x[x != 0]), _lowbits(w[w != 0])
    if lx.size == 0 or lw.size == 0:
        return True
    return bool((np.abs(x) @ np.abs(w).T).max() < 2.0 ** 24 * lx.min() * lw.min())


def fp8_blocks_exact(q: np.ndarray, w: np.ndarray) -> bool:
    """The FP8 MFMA adds the 128 products of a block exactly only when every product keeps its bits
    within 14 bits of the block's largest product (it truncates bits below 2^(e - 13), e the
    exponent of the largest product: measured 448 + 2^-9 -> 448, 64 + 7 * 2^-9 -> 64 + 2^-7).
    q [rows, K] and w [n, K] hold e4m3 values (without block scales): True when every block of every
    (row, output) sum is inside that window (a product's lowest bit is the product of its operands').

    Per block, cheap sufficient conditions come first: every output row of w has at most one nonzero
    (one product per sum), or, over the columns where some output row is nonzero, the smallest
    lowest bits of q's row and w's row times each other reach the window of the product of their
    largest magnitudes (an upper bound of the largest product). Pairs that neither settles are
    checked product by product."""
    lq, lw = _lowbits(q), _lowbits(w)
    for b in range(q.shape[1] // 128):
        blk = slice(128 * b, 128 * b + 128)
        wb = w[:, blk]
        if np.all(np.count_nonzero(wb, axis=1) <= 1):
            continue
        cols = np.any(wb != 0, axis=0)
        qb, wb = np.abs(q[:, blk][:, cols]), np.abs(wb[:, cols])
        lqb, lwb = lq[:, blk][:, cols], lw[:, blk][:, cols]
        qmin = np.where(lqb > 0, lqb, np.inf).min(axis=1)
        wmin = np.where(lwb > 0, lwb, np.inf).min(axis=1)
        bound = qb.max(axis=1)[:, None] * wb.max(axis=1)[None, :]
        live = bound > 0
        window = np.ldexp(1.0, np.floor(np.log2(np.where(live, bound, 1.0))).astype(np.int64) - 13)
        unsettled = live & (qmin[:, None] * wmin[None, :] < window)
        if not np.any(unsettled):
            continue
        rs, ns = np.nonzero(unsettled)
        for r, n in zip(rs, ns):
            prod = qb[r] * wb[n]
            mx = prod.max()
            if mx == 0:
                continue
            lp = lqb[r] * lwb[n]
            low = np.where(lp > 0, lp, np.inf).min()
            if low < np.ldexp(1.0, int(np.floor(np.log2(mx))) - 13):
                return False
    return True


def peak_offset(e, j):
    """Row, within hidden group j of expert e, of the closed-form layer's h = 448 entry."""
    return (41 * e + 67 * j + 5) % 128


def closed_form_mode_b(seed, rows, n_experts, hidden=256, inter=256, top_k=8, check=False, down_block_step=1):
    """A routed layer whose mode-B result is fixed bit for bit, whatever the summation order.

    Every activation group holds +-448 (so its dynamic scale is exactly 1 and the codes are the
    values), weights are e4m3 codes in [1, 2) times power-of-two block scales, and the columns that
    hold the +-448 entries carry no weight, so every gate/up sum is exact in f32. One hidden row of
    each 128-row group j of every expert, row 128 j + peak_offset(e, j) (spread over the whole group,
    so a group maximum taken over part of the group gets another scale), has gate 32 and up 14
    (silu(32) rounds to 32 in f32), so h = 448 there and every hidden group's scale is exactly 1
    too; the down weights skip those rows and hold one code per
    128-column block (hidden codes span e4m3's range, and one product per block keeps the FP8
    MFMA's block sums exact, see fp8_blocks_exact). Gate rows whose silu
    lies within 16 f32 steps of a bf16 rounding boundary are zeroed (an exp evaluated one step
    differently could round them the other way). Returns experts {id: (gw, gs, uw, us, dw, ds)},
    x [rows, hidden] f32, selected [rows, top_k], weights [rows, top_k]. With check, asserts that
    every projection sum of the routed placements is exact in f32 and inside the FP8 MFMA's window
    (a CPU test runs the checks for the seeds and sizes the GPU tests use). down_block_step: the
    down weights hold their one code per block only in every down_block_step-th 128-column block
    (zeros elsewhere), so that a wide intermediate keeps its down sums exact in f32."""
    rng = np.random.default_rng(seed)
    experts = {}
    for e in range(n_experts):
        gw, uw = _unit_codes(rng, (inter, hidden), 0.3), _unit_codes(rng, (inter, hidden), 0.3)
        dw = np.zeros((hidden, inter), np.uint8)
        for b in range(0, inter // 128, down_block_step):
            c = 128 * b + rng.integers(1, 128, hidden)
            dw[np.arange(hidden), c] = _unit_codes(rng, hidden, 0.0)
        for w in (gw, uw):
            w[:, 0] = 0
            w[:, 1::128] = 0
        gs = (2.0 ** rng.integers(-5, -3, (inter // 128, hidden // 128))).astype(np.float32)
        us = (2.0 ** rng.integers(-5, -3, (inter // 128, hidden // 128))).astype(np.float32)
        ds = (2.0 ** rng.integers(-5, -3, (hidden // 128, inter // 128))).astype(np.float32)
        for j in range(inter // 128):
            r = 128 * j + peak_offset(e, j)
            gw[r, :] = 0
            uw[r, :] = 0
            # x[:, 0] = 32: code * scale * 32 = 32 (gate) and 14 (up)
            gw[r, 0] = 0x58 if gs[j, 0] == 2.0 ** -4 else 0x60   # 16 or 32
            uw[r, 0] = 0x4E if us[j, 0] == 2.0 ** -4 else 0x56   # 7 or 14
            dw[:, r] = 0
        experts[e] = (gw, gs, uw, us, dw, ds)
    x = decode_table()[_unit_codes(rng, (rows, hidden), 0.2)].astype(np.float32)
    x[:, 0] = 32.0
    x[:, 1::128] = 448.0 * np.where(rng.random((rows, hidden // 128)) < 0.5, -1.0, 1.0)
    sel = np.stack([rng.permutation(n_experts)[:top_k] for _ in range(rows)]).astype(np.uint32)
    w = rng.uniform(0.05, 1.0, (rows, top_k)).astype(np.float32)
    w = (w / w.sum(axis=1, keepdims=True)).astype(np.float32)
    for e in sorted(set(sel.reshape(-1).tolist())):
        gw, gs, uw, us, dw, ds = experts[e]
        xs = x[[p for p in range(rows) if e in sel[p].tolist()]].astype(np.float64)
        if check:
            for wm, sm in ((gw, gs), (uw, us)):
                assert exact_in_f32(xs, dequant(wm, sm))
                assert fp8_blocks_exact(xs, decode_table()[wm])
        g = bf16_round((xs @ dequant(gw, gs).T).astype(np.float32)).astype(np.float64)
        silu = (g / (1.0 + np.exp(-g))).astype(np.float32)
        low = (silu.view(np.uint32) & 0xFFFF).astype(np.int64)
        near = np.any(np.abs(low - 0x8000) <= 16, axis=0)
        peaks = [128 * j + peak_offset(e, j) for j in range(inter // 128)]
        near[peaks] = False
        gw[near, :] = 0
        g = bf16_round((xs @ dequant(gw, gs).T).astype(np.float32)).astype(np.float64)
        u = bf16_round((xs @ dequant(uw, us).T).astype(np.float32)).astype(np.float32)
        h = bf16_round(bf16_round((g / (1.0 + np.exp(-g))).astype(np.float32)) * u).astype(np.float64)
        if check:
            assert np.all(np.abs(h[:, peaks]) == 448.0) and np.all(np.abs(h) <= 448.0)
            hd = decode_table()[encode_e4m3(h)]
            assert exact_in_f32(hd, dequant(dw, ds))
            assert fp8_blocks_exact(hd, decode_table()[dw])
    return experts, x, sel, w


def moe_condition(x, experts, sel, w):
    """Scale of the f32 summation-order error of a mode-A routed layer, per output [rows, hidden]:
    sum over the token's slots of |w| (|Wd| @ (|h| + |silu'(g) u| |Wg| |x| + |silu(g)| |Wu| |x|)),
    the sum of the magnitudes of every term whose rounding reaches the output (f64)."""
    x = np.asarray(x, np.float64)
    out = np.zeros(x.shape)
    for e in sorted(set(np.asarray(sel).reshape(-1).tolist())):
        gw, gs, uw, us, dw, ds = experts[e]
        rows_e = [p for p in range(x.shape[0]) if e in np.asarray(sel)[p].tolist()]
        xs = x[rows_e]
        wg, wu, wd = dequant(gw, gs), dequant(uw, us), dequant(dw, ds)
        g, u = xs @ wg.T, xs @ wu.T
        sig = 1.0 / (1.0 + np.exp(-g))
        silu = g * sig
        dsilu = sig * (1.0 + g * (1.0 - sig))
        ag, au = np.abs(xs) @ np.abs(wg).T, np.abs(xs) @ np.abs(wu).T
        inner = np.abs(silu * u) + np.abs(dsilu * u) * ag + np.abs(silu) * au
        cond = inner @ np.abs(wd).T
        for l, p in enumerate(rows_e):
            out[p] += abs(float(np.asarray(w)[p, np.asarray(sel)[p].tolist().index(e)])) * cond[l]
    return out


# Known-answer router rows that pin the route-weight denominator of pytorch_noaux_routes
# (src/text_endpoint.rs:4382-4390, :4450): w_i = s_i / (fold(0, +)(s0 + s4, s1 + s5, s2 + s6, s3 + s7)
# + 1e-20) over the selected scores in partition order. Each row is 256 logits, logit[e] =
# base - e / 256 except at `positions`, where logit = num / 256 (all exact in f32). Expected values are
# the reference's formula in IEEE f32; for each row the alternative orders listed in `differs` give
# other weight bits, so a slip to any of them fails.
#   tree      (l0 + l1) + (l2 + l3)
#   plain     s0 + s1 + ... + s7 left to right
#   id_order  the reference's fold over the selected scores taken in ascending expert id
#   no_eps    without the + 1e-20
ROUTE_WEIGHT_ROWS = [
    dict(base=-4.0, positions=[1, 3, 53, 76, 126, 169, 223, 236],
         num=[469, 210, 438, 481, 181, -41, -145, 176],
         selected=[53, 1, 76, 3, 126, 236, 169, 223],
         score_bits=[0x3f58d23b, 0x3f5cac43, 0x3f5e1387, 0x3f31bdd2, 0x3f2b7466, 0x3f2a5859, 0x3eeb8b31,
                     0x3eb960c7],
         weight_bits=[0x3e1fc77f, 0x3e229e1f, 0x3e23a6df, 0x3e02fb13, 0x3dfcb221, 0x3dfb0f7c, 0x3dad9383,
                      0x3d889bb7],
         differs=["tree", "plain", "id_order"]),
    dict(base=-40.0, positions=[130, 147, 148, 188, 194, 225, 236, 251],
         num=[-8031, -8362, -8373, -8301, -8229, -8335, -8193, -8184],
         selected=[251, 236, 188, 194, 130, 225, 147, 148],
         score_bits=[0x286b6112, 0x28633f77, 0x28150866, 0x28456fb7, 0x28d5f141, 0x28027f5b, 0x27eadebc,
                     0x27e0fde3],
         weight_bits=[0x3e16e310, 0x3e11acac, 0x3dbf1243, 0x3dfd20dd, 0x3e89252a, 0x3da74ec2, 0x3d968f83,
                      0x3d903a6c],
         differs=["tree", "plain", "id_order", "no_eps"]),
]


def route_weight_row_logits(row) -> np.ndarray:
    logits = (np.float32(row["base"]) - np.arange(256, dtype=np.float32) / np.float32(256)).astype(np.float32)
    logits[row["positions"]] = np.array(row["num"], np.float32) / np.float32(256)
    return logits


def route_weight_alternatives(scores_sel: np.ndarray, selected) -> dict:
    """Route weights of the selected scores (partition order) under the reference's denominator and
    under each alternative, in IEEE f32."""
    f = np.float32

    def lanes(s):
        return [f(s[0] + s[4]), f(s[1] + s[5]), f(s[2] + s[6]), f(s[3] + s[7])]

    def fold(s):
        acc = f(0.0)
        for v in lanes(s):
            acc = f(acc + v)
        return acc

    def plain(s):
        acc = f(0.0)
        for v in s:
            acc = f(acc + v)
        return acc

    def tree(s):
        ln = lanes(s)
        return f(f(ln[0] + ln[1]) + f(ln[2] + ln[3]))

    def weights(s, den, eps=True):
        d = f(den + f(1e-20)) if eps else den
        return np.array([f(v / d) for v in s], np.float32)

    s = np.asarray(scores_sel, np.float32)
    by_id = np.argsort(np.asarray(selected))
    s_id = s[by_id]
    return {
        "reference": weights(s, fold(s)),
        "tree": weights(s, tree(s)),
        "plain": weights(s, plain(s)),
        "id_order": weights(s, fold(s_id)),
        "no_eps": weights(s, fold(s), eps=False),
    }


# ------------------------------------------------------------------ staged SwiGLU known answers
# (gate bits, up bits) -> output bits of round(round(silu(round(g))) * round(u)). The expected
# outputs come from the exact silu (every case sits more than 64 f32 ulps from a bf16 rounding
# boundary, so any faithful f32 evaluation gives these bits). `dropped` is the output with the named
# rounding taken out; each differs from the expected bits.
STAGED_CASES = [
    # the reference's case: gate 1.03125, up 0.71484375 (src/staged_metal_expert.rs:2826-2831)
    dict(g=0x3F840000, u=0x3F370000, out=0x3F0B0000, dropped={}),
    # silu rounding: 0.9913 * -1.3032
    dict(g=0x3F7DC693, u=0xBFA6CDDB, out=0xBF710000, dropped={"silu": 0xBF720000}),
    # up rounding: 1.0937 * 0.2941
    dict(g=0x3F8BFEED, u=0x3E969889, out=0x3E780000, dropped={"up": 0x3E770000}),
    # gate rounding: 0.02443 * -0.2756
    dict(g=0x3CC81A2C, u=0xBE8D1BD3, out=0xBB5F0000, dropped={"gate": 0xBB600000}),
    # product exactly halfway between two bf16 values (0xbd968000): ties to the even code
    dict(g=0xC02E0000, u=0x3EE00000, out=0xBD960000, dropped={"product": 0xBD968000}),
]
STAGES = ("gate", "up", "silu", "product")


def staged_swiglu_independent(g_bits, u_bits, drop=None):
    """The staged SwiGLU evaluated independently of the oracle, with the stage `drop` left unrounded:
    bf16 rounding in numpy, silu in f64 (math.exp) rounded once to f32, the product in f32."""
    def rnd(v, stage):
        return v if stage == drop else np.float32(bf16_round(np.array([v], np.float32))[0])

    g = rnd(np.float32(np.uint32(g_bits).view(np.float32)), "gate")
    u = rnd(np.float32(np.uint32(u_bits).view(np.float32)), "up")
    silu = rnd(np.float32(float(g) / (1.0 + math.exp(-float(g)))), "silu")
    return int(np.float32(rnd(np.float32(silu * u), "product")).view(np.uint32))
