"""Writes tests/golden/moe_small.npz: small seeded inputs of the MoE block's functions and their expected
outputs, computed here by brute force in Python / numpy float64, independently of oracle/ (which uses torch).

    python tests/golden/make_fixtures.py

What the expectations restate, and from where (paths relative to the Ming Voice sources):
  align     fused_moe.py:154-173 _align_blocks: pairs grouped by expert in ascending pair order, each
            expert's run padded to a multiple of BM with the pad value P; bexp per block, -1 past the used
            blocks; nb = ceil((P + E1 * (BM - 1)) / BM). Computed with Python lists, one pair at a time.
  quantize  fused_moe.py:199-204 quantize_rows_int8: scale = max(|w|, 1e-8) / 127 per row (fp32),
            q = round-half-even(w / scale) clamped to [-127, 127]. Computed per element in float64 with
            the fp32 roundings made explicit.
  select    the configs' softmax router: top-k of logits + bias (ties: lowest expert first, by a Python
            sort on (-key, index)), weights = softmax over all experts, renormalised over the picks; the
            shared expert E appended with weight 1.
  moe       fused_moe.py:13-61 (one token per expert slot): g = bf16(x . Wg), u = bf16(x . Wu),
            a = bf16(bf16(silu(g)) * u), part = bf16(a . Wd), y = bf16(sum_k w_k * part_k) + x rounded
            to bf16; dot products in float64 (the kernels' fp32 sums differ from these by far less than
            one bf16 ulp at these sizes, so the tests compare with the bf16 tolerance).
  moe int8  the same block with the experts quantised per row with bf16 scales (engine.py:126-147 with
            quantize_rows_int8, scale rounded to bf16 and q = round(w / scale)); fused_moe.py:34-38,
            60-61: the row scale multiplies the float64 accumulator before each bf16 rounding.
bf16 rounding is done on the float32 bit pattern (round to nearest, ties to even) with numpy integers.
"""
import math
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
OUT = os.path.join(HERE, "moe_small.npz")


def f32(v):
    return float(np.float32(v))


def bf16(v):
    """float -> nearest bf16 value (ties to even), returned as a Python float."""
    b = np.array([v], dtype=np.float32).view(np.uint32)[0]
    b = int(b)
    b = (b + 0x7FFF + ((b >> 16) & 1)) & 0xFFFF0000
    return float(np.array([b], dtype=np.uint32).view(np.float32)[0])


def bf16_array(a):
    return np.array([bf16(v) for v in np.asarray(a, dtype=np.float64).ravel()], dtype=np.float32).reshape(np.shape(a))


def align(flat, E1, BM):
    P = len(flat)
    per = [[] for _ in range(E1)]
    for p, e in enumerate(flat):
        if 0 <= e < E1:
            per[e].append(p)
    nb = (P + E1 * (BM - 1) + BM - 1) // BM
    sorted_ids, bexp, offsets = [], [], [0]
    for e in range(E1):
        if per[e]:
            rows = per[e] + [P] * ((-len(per[e])) % BM)
            sorted_ids += rows
            bexp += [e] * (len(rows) // BM)
        offsets.append(len(sorted_ids))
    sorted_ids += [P] * (nb * BM - len(sorted_ids))
    bexp += [-1] * (nb - len(bexp))
    return np.array(sorted_ids, np.int32), np.array(bexp, np.int32), np.array(offsets, np.int32)


def quantize(w):
    q = np.zeros(w.shape, np.int8)
    s = np.zeros(w.shape[0], np.float32)
    for r in range(w.shape[0]):
        amax = max(max(abs(float(v)) for v in w[r]), 1e-8)
        scale = f32(f32(amax) / 127.0)
        s[r] = scale
        for c in range(w.shape[1]):
            t = f32(float(w[r, c]) / scale)  # fp32 division, as the reference's w / scale
            k = round(t)  # Python rounds half to even
            q[r, c] = max(-127, min(127, k))
    return q, s


def quantize_bf16_scales(w):
    """Rows of w (last dim) -> (q int8, scale as bf16 values): scale = bf16(max(|w|, 1e-8) / 127) and
    q = round-half-even(w / scale) clamped to [-127, 127], the division in fp32."""
    flat = w.reshape(-1, w.shape[-1])
    q = np.zeros(flat.shape, np.int8)
    sc = np.zeros(flat.shape[0], np.float32)
    for r in range(flat.shape[0]):
        amax = max(max(abs(float(v)) for v in flat[r]), 1e-8)
        scale = bf16(f32(f32(amax) / 127.0))
        sc[r] = scale
        for c in range(flat.shape[1]):
            q[r, c] = max(-127, min(127, round(f32(float(flat[r, c]) / scale))))
    return q.reshape(w.shape), sc.reshape(w.shape[:-1])


def select(logits, bias, top_k, E):
    N = logits.shape[0]
    ids = np.zeros((N, top_k + 1), np.int64)
    wts = np.zeros((N, top_k + 1), np.float32)
    for t in range(N):
        key = [float(logits[t, e]) + float(bias[e]) for e in range(E)]
        order = sorted(range(E), key=lambda e: (-key[e], e))[:top_k]
        m = max(key)
        ex = [math.exp(k - m) for k in key]
        den = sum(ex)
        p = [v / den for v in ex]
        tot = sum(p[e] for e in order)
        for k, e in enumerate(order):
            ids[t, k] = e
            wts[t, k] = p[e] / (tot + 1e-20)
        ids[t, top_k] = E
        wts[t, top_k] = 1.0
    return ids, wts


def moe(x, w_gu, w_d, ids, wts, s_gu=None, s_d=None):
    N, H = x.shape
    I = w_d.shape[-1]
    y = np.zeros((N, H), np.float32)
    a_rows = np.zeros((N * ids.shape[1], I), np.float32)
    one = lambda *_: 1.0  # noqa: E731
    sg = (lambda e, r: float(s_gu[e, r])) if s_gu is not None else one
    sd = (lambda e, h: float(s_d[e, h])) if s_d is not None else one
    for t in range(N):
        acc = np.zeros(H, np.float64)
        for k in range(ids.shape[1]):
            e = int(ids[t, k])
            g = [bf16(sum(float(x[t, h]) * float(w_gu[e, r, h]) for h in range(H)) * sg(e, r)) for r in range(I)]
            u = [bf16(sum(float(x[t, h]) * float(w_gu[e, I + r, h]) for h in range(H)) * sg(e, I + r))
                 for r in range(I)]
            a = [bf16(bf16(gg / (1.0 + math.exp(-gg))) * uu) for gg, uu in zip(g, u)]
            a_rows[t * ids.shape[1] + k] = a
            part = [bf16(sum(a[r] * float(w_d[e, h, r]) for r in range(I)) * sd(e, h)) for h in range(H)]
            acc += float(wts[t, k]) * np.array(part, np.float64)
        y[t] = [bf16(bf16(v) + float(x[t, h])) for h, v in enumerate(acc)]
    return y, a_rows


def main():
    rng = np.random.default_rng(20261202)
    fx = {}
    # align: ragged, with an out-of-range id, two block heights
    flat = rng.integers(0, 9, size=50)
    flat[[3, 17]] = [9, -1]  # dropped pairs
    fx["align_flat"] = flat.astype(np.int64)
    for bm in (4, 64):
        s, b, o = align(list(flat), 9, bm)
        fx[f"align_sorted_bm{bm}"], fx[f"align_bexp_bm{bm}"], fx[f"align_offsets_bm{bm}"] = s, b, o
    # quantize: bf16-valued rows, one zero row, one row with a .5 tie after scaling
    w = bf16_array(rng.normal(0.0, 0.02, size=(6, 64)))
    w[2] = 0.0
    w[4, :] = 0.0  # amax 127/64 makes the scale exactly 1/64: w = k.5/64 lands on a tie (half to even)
    w[4, :4] = [127.0 / 64, 2.5 / 64, -3.5 / 64, 0.5 / 64]  # q = 127, 2, -4, 0
    fx["quant_w"] = w
    fx["quant_q"], fx["quant_s"] = quantize(w)
    # router selection (softmax top-3 of 8 experts + shared), with an exact tie
    logits = rng.normal(0.0, 1.0, size=(5, 8)).astype(np.float32)
    logits[1, 2] = logits[1, 5] = 3.0
    bias = rng.normal(0.0, 0.5, size=8).astype(np.float32)
    fx["sel_logits"], fx["sel_bias"] = logits, bias
    fx["sel_ids"], fx["sel_wts"] = select(logits, bias, 3, 8)
    # one MoE block: H=64, I=32, 4 routed experts + shared, 3 tokens, top-2 + shared
    H, I, E = 64, 32, 4
    x = bf16_array(rng.normal(0.0, 1.0, size=(3, H)))
    w_gu = bf16_array(rng.normal(0.0, 0.05, size=(E + 1, 2 * I, H)))
    w_d = bf16_array(rng.normal(0.0, 0.05, size=(E + 1, H, I)))
    ids = np.array([[0, 2, E], [3, 1, E], [2, 0, E]], np.int64)
    wts = np.array([[0.6, 0.4, 1.0], [0.7, 0.3, 1.0], [0.5, 0.5, 1.0]], np.float32)
    fx["moe_x"], fx["moe_w_gu"], fx["moe_w_d"], fx["moe_ids"], fx["moe_wts"] = x, w_gu, w_d, ids, wts
    fx["moe_y"], fx["moe_a"] = moe(x, w_gu, w_d, ids, wts)
    # the same block on int8 experts with bf16 row scales
    q_gu, s_gu = quantize_bf16_scales(w_gu)
    q_d, s_d = quantize_bf16_scales(w_d)
    fx["moe_q_gu"], fx["moe_s_gu"], fx["moe_q_d"], fx["moe_s_d"] = q_gu, s_gu, q_d, s_d
    fx["moe_y_i8"], fx["moe_a_i8"] = moe(x, q_gu, q_d, ids, wts, s_gu, s_d)
    np.savez_compressed(OUT, **fx)
    print(f"wrote {OUT} ({os.path.getsize(OUT)} bytes)")


if __name__ == "__main__":
    main()
