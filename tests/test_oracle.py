"""Pins of the CPU oracle: reference-held tests restated, closed forms,
brute force and invariants.  CPU only."""
import numpy as np
import pytest


# ------------------------------------------------------------ quantize
@pytest.mark.parametrize("bits", [2, 4, 8])
def test_quantize_dequantize_reference_bound(orc, bits):
    """crates/mlxr/src/ops/quantization.rs:299-315: rows arange(0, 512) at
    group 128; shapes, and max |x - x_hat| <= 127 / 2^bits."""
    x = np.broadcast_to(np.arange(0, 512, dtype=np.float32), (128, 512)).copy()
    wq, sc, bi = orc.quantize(x, group_size=128, bits=bits, bf16=False)
    assert wq.shape == (128, 512 // (32 // bits))
    assert sc.shape == (128, 4) and bi.shape == (128, 4)
    xh = orc.dequantize(wq, sc, bi, group_size=128, bits=bits, out_bf16=False)
    assert np.abs(x - xh).max() <= 127.0 / (1 << bits)


def test_quantize_constant_group_is_exact(orc):
    w = np.full((3, 64), 0.5, np.float32)
    w[1] = -2.25
    w[2] = 0.0
    wq, sc, bi = orc.quantize(w, 64, 4, bf16=False)
    assert np.array_equal(orc.dequantize(wq, sc, bi, 64, 4, out_bf16=False), w)


@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("sign", [1.0, -1.0])
def test_quantize_exact_ladder(orc, bits, sign):
    """A group that is exactly bias + k * step for every code k is
    reconstructed exactly (edge snapping: the larger-magnitude end is
    code 0)."""
    n = 1 << bits
    step = 0.25
    rng = np.random.default_rng(bits)
    codes = np.concatenate([[0, n - 1], rng.integers(0, n, 62)]).astype(np.float32)
    w = (sign * (codes * step - 1.0)).astype(np.float32)[None, :]
    wq, sc, bi = orc.quantize(w, 64, bits, bf16=False)
    assert np.array_equal(orc.dequantize(wq, sc, bi, 64, bits, out_bf16=False), w)
    edge = w[0, np.argmax(np.abs(w[0]))]
    assert bi[0, 0] == edge


@pytest.mark.parametrize("bits", [2, 4, 8])
def test_quantize_codes_are_nearest(orc, bits):
    """Brute force over all codes: each code minimises |w - (q*s + b)| for
    the group's (f32-stored, so unrounded) scale and bias."""
    rng = np.random.default_rng(1)
    w = (rng.standard_normal((16, 128)) * 0.02).astype(np.float32)
    wq, sc, bi = orc.quantize(w, 64, bits, bf16=False)
    per = 32 // bits
    codes = ((wq[:, :, None] >> (np.arange(per, dtype=np.uint32) * bits)) & ((1 << bits) - 1))
    codes = codes.reshape(16, 128).astype(np.float64)
    s = np.repeat(sc.astype(np.float64), 64, axis=1)
    b = np.repeat(bi.astype(np.float64), 64, axis=1)
    err = np.abs(w - (codes * s + b))
    allq = np.arange(1 << bits, dtype=np.float64)
    best = np.abs(w[:, :, None] - (allq * s[:, :, None] + b[:, :, None])).min(-1)
    assert np.all(err <= best + 1e-6 * np.abs(s))
    # edge snapping: the bias is the group's larger-magnitude end and sits
    # an integer number of scales from zero
    g = w.reshape(16, 2, 64)
    edge = np.take_along_axis(g, np.abs(g).argmax(-1)[..., None], -1)[..., 0]
    assert np.array_equal(bi, edge)
    q0 = bi.astype(np.float64) / sc.astype(np.float64)
    assert np.all(np.abs(q0 - np.rint(q0)) <= 1e-5 * np.abs(q0))
    assert np.all((q0 <= 0) & (np.abs(q0) <= (1 << bits) - 1 + 0.5))


def test_dequantize_slot_layout(orc):
    """kernel_source.rs:101-104: slot j of a word holds bits [j*b, (j+1)*b);
    dequant = code * scale + bias (one rounding)."""
    rng = np.random.default_rng(2)
    for bits in (2, 4, 8):
        per = 32 // bits
        codes = rng.integers(0, 1 << bits, size=(4, 64), dtype=np.uint32)
        words = np.zeros((4, 64 // per), np.uint32)
        for j in range(per):
            words |= codes[:, j::per] << np.uint32(j * bits)
        sc = orc.f32_to_bf16(rng.standard_normal((4, 1)).astype(np.float32) * 0.01)
        bi = orc.f32_to_bf16(rng.standard_normal((4, 1)).astype(np.float32) * 0.1)
        got = orc.dequantize(words, sc, bi, 64, bits, out_bf16=True)
        exact = codes.astype(np.float64) * orc.bf16_to_f32(sc).astype(np.float64) + \
            orc.bf16_to_f32(bi).astype(np.float64)
        want = orc.f32_to_bf16(exact.astype(np.float32))
        assert np.array_equal(got, want), bits


def test_quantize_bf16_storage_round_trip(orc):
    rng = np.random.default_rng(3)
    w = orc.f32_to_bf16((rng.standard_normal((8, 256)) * 0.02).astype(np.float32))
    wq, sc, bi = orc.quantize(w, 64, 4, bf16=True)
    wh = orc.bf16_to_f32(orc.dequantize(wq, sc, bi, 64, 4))
    wf = orc.bf16_to_f32(w)
    s = np.abs(np.repeat(orc.bf16_to_f32(sc), 64, axis=1))
    b = np.abs(np.repeat(orc.bf16_to_f32(bi), 64, axis=1))
    # Snapping the edge to an exact code stretches the grid by at most
    # 0.5/|q0| (|q0| >= 7.5 at 4 bits), so the far end can overshoot the
    # last code by up to one step; plus the bf16 rounding of the scale
    # (times the code, at most 15), of the bias and of the result.
    bound = 1.0 * s + (15 * s + b + np.abs(wh)) * 2.0 ** -8
    assert np.all(np.abs(wh - wf) <= bound)


def test_quantize_edge_snap_closed_form(orc):
    """MLX's affine recipe on a hand-computed group (4 bits, n_bins 15):
    max 1.0, min m with (1 - m) = 15 / 7.7, so the unsnapped scale is
    s0 = -(1 - m) / 15 and edge / s0 = -7.7.  The edge snaps to the
    nearest code, q0 = -8 (a truncation would give -7), so the stored
    scale is exactly 1 / -8 = -0.125 and the bias the edge, 1.0."""
    w = np.zeros((1, 64), np.float32)
    m = np.float32(1.0) - np.float32(15.0 / 7.7)
    w[0, 0] = 1.0
    w[0, 1] = m
    w[0, 2:] = np.linspace(m, 1.0, 62, dtype=np.float32)
    s0 = -((np.float32(1.0) - m) / np.float32(15.0))
    assert -7.71 < np.float32(1.0) / s0 < -7.69  # the fraction rint and trunc split on
    wq, sc, bi = orc.quantize(w, 64, 4, bf16=False)
    assert sc[0, 0] == np.float32(-0.125) and bi[0, 0] == np.float32(1.0)
    codes = (wq[0, :, None] >> (np.arange(8, dtype=np.uint32) * 4)) & 15
    codes = codes.reshape(-1)
    # the edge is code 0; the far end (m - 1) / -0.125 = 15.58 clamps to 15
    assert codes[0] == 0 and codes[1] == 15
    # and a negative edge: the same group mirrored snaps to +8 with bias -1
    wq, sc, bi = orc.quantize(-w, 64, 4, bf16=False)
    assert sc[0, 0] == np.float32(0.125) and bi[0, 0] == np.float32(-1.0)


@pytest.mark.parametrize("bits", [4, 8])
def test_quantize_edge_snaps_to_nearest_code(orc, bits):
    """For every group, q0 = bias / scale is the integer nearest to
    edge / s0, with s0 = -+max((max - min) / n_bins, 1e-7) the unsnapped
    scale (sign towards the smaller-magnitude end), both in f32.  Groups are
    drawn so edge / s0 spans many fractions, both sides of one half."""
    rng = np.random.default_rng(11 + bits)
    n_bins = np.float32((1 << bits) - 1)
    rows = 512
    hi = rng.uniform(0.5, 2.0, rows).astype(np.float32)
    lo = -hi * rng.uniform(0.0, 1.0, rows).astype(np.float32)
    sign = np.where(rng.random(rows) < 0.5, 1.0, -1.0).astype(np.float32)
    w = (rng.uniform(0, 1, (rows, 64)).astype(np.float32) * (hi - lo)[:, None] + lo[:, None])
    w[:, 0], w[:, 1] = hi, lo
    w *= sign[:, None]
    wq, sc, bi = orc.quantize(w, 64, bits, bf16=False)
    wmax, wmin = w.max(1), w.min(1)
    neg = np.abs(wmin) > np.abs(wmax)
    s0 = np.maximum((wmax - wmin) / n_bins, np.float32(1e-7)).astype(np.float32)
    s0 = np.where(neg, s0, -s0).astype(np.float32)
    edge = np.where(neg, wmin, wmax).astype(np.float32)
    ratio = (edge / s0).astype(np.float64)
    frac = np.abs(ratio - np.trunc(ratio))
    assert (frac > 0.5).sum() > 50 and (frac < 0.5).sum() > 50
    q0 = np.rint(bi[:, 0].astype(np.float64) / sc[:, 0].astype(np.float64))
    assert np.all(np.abs(q0 - ratio) <= 0.5)
    assert np.array_equal(bi[:, 0], edge)


def test_quantize_rejects_bad_args(orc):
    with pytest.raises(ValueError):
        orc.quantize(np.zeros((2, 64), np.float32), 64, 3, bf16=False)
    with pytest.raises(ValueError):
        orc.quantize(np.zeros((2, 96), np.float32), 64, 4, bf16=False)


# -------------------------------------------------------------- router
def test_router_logits_rounding_bound(orc):
    rng = np.random.default_rng(4)
    T, d, E = 5, 2048, 16
    x = orc.f32_to_bf16(rng.standard_normal((T, d)).astype(np.float32))
    w = (rng.standard_normal((E, d)) * 0.02).astype(np.float32)
    got = orc.router_logits(x, w).astype(np.float64)
    xf = orc.bf16_to_f32(x).astype(np.float64)
    exact = xf @ w.astype(np.float64).T
    bound = d * 2.0 ** -23 * (np.abs(xf) @ np.abs(w.astype(np.float64)).T)
    assert np.all(np.abs(got - exact) <= bound)
    # experts are independent: permuting rows permutes columns bit-exactly
    perm = rng.permutation(E)
    assert np.array_equal(orc.router_logits(x, w[perm]), got.astype(np.float32)[:, perm])


def test_router_logits_one_hot(orc):
    d, E = 512, 8
    w = np.random.default_rng(5).standard_normal((E, d)).astype(np.float32)
    for j in (0, 3, 255, 511):
        x = np.zeros((1, d), np.float32)
        x[0, j] = 1.0
        assert np.array_equal(orc.router_logits(orc.f32_to_bf16(x), w)[0], w[:, j])


def test_router_logits_mfma_order(orc):
    """The matrix-core order (router_logits(mfma=True)), pinned by values
    whose sum depends on the order: 2^24 + 1 rounds back to 2^24 in f32,
    so a term of 1 survives only where it is added after the +-2^24 pair
    has cancelled.  Within a 16-element chunk the order is j, j+8, j+1,
    j+9, ...: w[0] = 2^24, w[8] = 1, w[1] = -2^24 loses the 1 (0), where
    the natural order j, j+1, ... would keep it (1).  Across quarters the
    sum is ((q0 + q1) + q2) + q3: q0 = 2^24, q1 = 1, q2 = -2^24 gives 0,
    where (q0 + q2) + q1 would give 1."""
    d = 256
    x = orc.f32_to_bf16(np.ones((1, d), np.float32))
    w = np.zeros((2, d), np.float32)
    w[0, 0], w[0, 8], w[0, 1] = 2.0 ** 24, 1.0, -(2.0 ** 24)
    w[1, 0], w[1, 64], w[1, 128] = 2.0 ** 24, 1.0, -(2.0 ** 24)
    assert orc.router_logits(x, w, mfma=True)[0].tolist() == [0.0, 0.0]
    # the lane order sums those elements otherwise (1 survives in row 0)
    assert orc.router_logits(x, w)[0, 0] == 1.0
    # the last element of a chunk comes after its pair: w[7] then w[15]
    w2 = np.zeros((1, d), np.float32)
    w2[0, 7], w2[0, 15], w2[0, 16] = 2.0 ** 24, 1.0, -(2.0 ** 24)
    assert orc.router_logits(x, w2, mfma=True)[0, 0] == 0.0
    w2[0, 15], w2[0, 16] = -(2.0 ** 24), 1.0   # cancel first, then add 1
    assert orc.router_logits(x, w2, mfma=True)[0, 0] == 1.0


def test_router_logits_mfma_bound_and_one_hot(orc):
    """The matrix-core order is an f32 dot product like the lane order: the
    rounding bound against fp64, experts independent, one-hot inputs exact,
    and d off a multiple of 64 refused."""
    rng = np.random.default_rng(14)
    T, d, E = 5, 2048, 16
    x = orc.f32_to_bf16(rng.standard_normal((T, d)).astype(np.float32))
    w = (rng.standard_normal((E, d)) * 0.02).astype(np.float32)
    got = orc.router_logits(x, w, mfma=True).astype(np.float64)
    xf = orc.bf16_to_f32(x).astype(np.float64)
    exact = xf @ w.astype(np.float64).T
    bound = d * 2.0 ** -23 * (np.abs(xf) @ np.abs(w.astype(np.float64)).T)
    assert np.all(np.abs(got - exact) <= bound)
    perm = rng.permutation(E)
    assert np.array_equal(orc.router_logits(x, w[perm], mfma=True),
                          got.astype(np.float32)[:, perm])
    for j in (0, 9, 513, 2047):
        xo = np.zeros((1, d), np.float32)
        xo[0, j] = 1.0
        assert np.array_equal(orc.router_logits(orc.f32_to_bf16(xo), w, mfma=True)[0],
                              w[:, j])
    with pytest.raises(ValueError):
        orc.router_logits(orc.f32_to_bf16(np.ones((1, 96), np.float32)),
                          np.ones((2, 96), np.float32), mfma=True)


def test_router_topk_matches_full_sort(orc):
    rng = np.random.default_rng(6)
    T, E, K = 64, 8, 2
    lg = rng.standard_normal((T, E)).astype(np.float32)
    lg[0, :] = 0.25  # all tied: lowest ids win
    lg[1, 5] = lg[1, 2] = lg[1].max() + 1.0
    idx, w = orc.router_topk(lg, K)
    for t in range(T):
        order = sorted(range(E), key=lambda e: (-float(lg[t, e]), e))
        assert list(idx[t]) == order[:K]
    p = np.exp(lg.astype(np.float64) - lg.max(1, keepdims=True))
    p /= p.sum(1, keepdims=True)
    pk = np.take_along_axis(p, idx, 1)
    assert np.allclose(w, pk / pk.sum(1, keepdims=True), rtol=1e-6, atol=1e-7)
    assert np.allclose(w.sum(1), 1.0, atol=1e-6)
    assert list(idx[0]) == [0, 1]
    assert list(idx[1]) == [2, 5]


# ---------------------------------------------- quantised (bf16) router
@pytest.mark.parametrize("bits", [4, 8, 16])
def test_router_logits_q_mfma_is_dequant_then_bf16(orc, bits):
    """The quantised (and bf16) router in the matrix-core order: the f32
    router's matrix-core order on the f32-dequantised weights (bits 16: the
    bf16 values), rounded once to bf16 -- and unlike the lane order's
    rounding on inputs where the two orders' f32 sums differ."""
    rng = np.random.default_rng(50 + bits)
    T, d, E = 6, 2048, 16
    x = orc.f32_to_bf16(rng.standard_normal((T, d)).astype(np.float32))
    w = orc.f32_to_bf16((rng.standard_normal((E, d)) * 0.02).astype(np.float32))
    if bits == 16:
        wq, sc, bi, wd = w, None, None, orc.bf16_to_f32(w)
    else:
        wq, sc, bi = orc.quantize(w, 64, bits)
        wd = orc.dequantize(wq, sc, bi, 64, bits, out_bf16=False)
    got = orc.router_logits_q(x, wq, sc, bi, bits, mfma=True)
    want = orc.bf16_to_f32(orc.f32_to_bf16(orc.router_logits(x, wd, mfma=True)))
    assert np.array_equal(got, want)
    # the order reaches the result: pre-rounding f32 sums differ somewhere
    assert not np.array_equal(orc.router_logits(x, wd, mfma=True), orc.router_logits(x, wd))


@pytest.mark.parametrize("bits", [4, 8])
def test_router_logits_q_is_dequant_then_bf16(orc, bits):
    """QuantizedLinear router (layers/quantized.rs:356-373): the f32 router
    on the f32-dequantised weights (same lane order), rounded once to bf16;
    within half a bf16 ulp (plus the f32 accumulation bound) of the fp64
    product."""
    rng = np.random.default_rng(40 + bits)
    T, d, E = 6, 2048, 16
    x = orc.f32_to_bf16(rng.standard_normal((T, d)).astype(np.float32))
    w = orc.f32_to_bf16((rng.standard_normal((E, d)) * 0.02).astype(np.float32))
    wq, sc, bi = orc.quantize(w, 64, bits)
    got = orc.router_logits_q(x, wq, sc, bi, bits)
    wd = orc.dequantize(wq, sc, bi, 64, bits, out_bf16=False)
    want = orc.bf16_to_f32(orc.f32_to_bf16(orc.router_logits(x, wd)))
    assert np.array_equal(got, want)
    xf = orc.bf16_to_f32(x).astype(np.float64)
    exact = xf @ wd.astype(np.float64).T
    bound = (d * 2.0 ** -23 * (np.abs(xf) @ np.abs(wd.astype(np.float64)).T)
             + 2.0 ** -8 * np.abs(exact))
    assert np.all(np.abs(got - exact) <= bound)
    # a one-hot row picks the dequantised weight column, rounded to bf16
    x1 = np.zeros((1, d), np.float32)
    x1[0, 777] = 1.0
    col = orc.router_logits_q(orc.f32_to_bf16(x1), wq, sc, bi, bits)[0]
    assert np.array_equal(col, orc.bf16_to_f32(orc.f32_to_bf16(wd[:, 777])))


def test_router_topk_bf16_selects_on_bf16_probs(orc):
    """softmax of bf16 logits is bf16 (arithmetic.rs:1298-1311) and
    argpartition selects on it: a full sort of the bf16 probabilities of
    the exact softmax, ties to the lower id -- also where the logits
    differ."""
    rng = np.random.default_rng(41)
    T, E, K = 64, 8, 3
    lg = orc.bf16_to_f32(orc.f32_to_bf16(rng.standard_normal((T, E)).astype(np.float32)))
    lg[0, :] = 0.5                       # all tied
    lg[1, :] = -6.0                      # distinct logits, equal bf16 probabilities:
    lg[1, 6] = 0.0                       # exp(2^-10) - 1 = 0.1% is well below one
    lg[1, 4] = 2.0 ** -10                # bf16 step of p ~ 0.5
    lg = lg.astype(np.float32)
    idx, w = orc.router_topk_bf16(lg, K)
    p = np.exp(lg.astype(np.float64) - lg.max(1, keepdims=True))
    p /= p.sum(1, keepdims=True)
    pb = orc.bf16_to_f32(orc.f32_to_bf16(p.astype(np.float32)))
    assert np.all(np.abs(pb - p) <= 2.0 ** -8 * p)
    for t in range(T):
        order = sorted(range(E), key=lambda e: (-float(pb[t, e]), e))
        assert list(idx[t]) == order[:K]
    assert list(idx[0]) == [0, 1, 2]
    assert pb[1, 4] == pb[1, 6] and lg[1, 6] < lg[1, 4]
    assert list(idx[1][:2]) == [4, 6] and pb[1, 4] == pb[1, 6]
    # bf16 weights within two bf16 roundings of the renormalised top-K
    pk = np.take_along_axis(pb, idx, 1).astype(np.float64)
    exact = pk / pk.sum(1, keepdims=True)
    assert np.all(np.abs(w - exact) <= 2.0 ** -7 * exact)
    assert np.array_equal(w, orc.bf16_to_f32(orc.f32_to_bf16(w)))


def test_combine_bf16_per_op_rounding(orc):
    """w * y, the sum over k and the shared branch each rounded to bf16
    (MLX evaluates bf16 ops in the arrays' dtype), restated elementwise."""
    rng = np.random.default_rng(42)
    T, K, d = 5, 4, 128
    bf = lambda a: orc.bf16_to_f32(orc.f32_to_bf16(np.asarray(a, np.float32)))
    y = orc.f32_to_bf16(rng.standard_normal((T, K, d)).astype(np.float32))
    w = bf(rng.random((T, K)))
    sy = orc.f32_to_bf16(rng.standard_normal((T, d)).astype(np.float32))
    sl = bf(rng.standard_normal(T))
    got = orc.bf16_to_f32(orc.combine_bf16(y, w, sy, sl))
    want = np.zeros((T, d), np.float32)
    for t in range(T):
        acc = np.zeros(d, np.float32)
        for k in range(K):
            acc = (acc + bf(w[t, k] * orc.bf16_to_f32(y[t, k]))).astype(np.float32)
        gate = bf(np.float32(1.0) / (np.float32(1.0) + np.exp(np.float32(-sl[t]))))
        want[t] = bf(bf(orc.bf16_to_f32(sy[t]) * gate) + bf(acc))
    assert np.array_equal(got, want)
    # against the f32 combine: K + 1 bf16 roundings of terms bounded by
    # sum_k |w_k y_k|
    routed = orc.bf16_to_f32(orc.combine_bf16(y, w)).astype(np.float64)
    mag = np.einsum("tk,tkd->td", np.abs(w), np.abs(orc.bf16_to_f32(y))).astype(np.float64)
    assert np.all(np.abs(routed - orc.combine(y, w)) <= (K + 1) * 2.0 ** -8 * mag)


def test_shared_gate_closed_forms(orc):
    """The shared branch is y_s * sigmoid(g) (moe.rs:118-120,145).  At
    g = 0 the gate is exactly 1/2, at g = 40 it is 1 in f32 and at g = -40
    it is ~4e-18, so out = routed + y_s / 2, routed + y_s and routed, each
    exact in f32 (halving is exact); the bf16 combine the same with each
    sum rounded once to bf16."""
    rng = np.random.default_rng(5)
    T, K, d = 3, 4, 64
    y = orc.f32_to_bf16(rng.standard_normal((T, K, d)).astype(np.float32))
    w = rng.random((T, K)).astype(np.float32)
    sy = orc.f32_to_bf16(rng.standard_normal((T, d)).astype(np.float32))
    ys = orc.bf16_to_f32(sy)
    routed = orc.combine(y, w)
    assert np.all(routed != 0)
    sl = np.array([0.0, 40.0, -40.0], np.float32)
    got = orc.combine(y, w, sy, sl)
    assert np.array_equal(got[0], (routed[0] + np.float32(0.5) * ys[0]).astype(np.float32))
    assert np.array_equal(got[1], (routed[1] + ys[1]).astype(np.float32))
    assert np.array_equal(got[2], routed[2])
    # bf16 weights: out = bf16(bf16(y_s * gate) + bf16(routed sum))
    bf = lambda a: orc.bf16_to_f32(orc.f32_to_bf16(np.asarray(a, np.float32)))
    wb = bf(w)
    rb = orc.bf16_to_f32(orc.combine_bf16(y, wb))
    gotb = orc.bf16_to_f32(orc.combine_bf16(y, wb, sy, sl))
    assert np.array_equal(gotb[0], bf(rb[0] + bf(np.float32(0.5) * ys[0])))
    assert np.array_equal(gotb[1], bf(rb[1] + ys[1]))
    assert np.array_equal(gotb[2], rb[2])
    # sigma(ln 3) = 3/4: within one f32 rounding of the gate
    g = np.array([np.log(3.0)] * T, np.float32)
    d3 = orc.combine(y, w, sy, g).astype(np.float64) - routed
    assert np.allclose(d3, 0.75 * ys, rtol=2e-6, atol=1e-6 * np.abs(routed).max())


@pytest.mark.parametrize("router_bits", [0, 8])
def test_block_shared_branch_fp64(orc, router_bits):
    """A block with a shared expert minus the same block without it (same
    router, so the same routing) is sigmoid(x . g_s) * shared(x), checked
    against an fp64 evaluation: the dequantised shared weights, matmuls
    and the sigmoid in double, no intermediate roundings.  The bound
    covers the bf16 rounding points of the reference's op sequence
    (gather_qmm outputs, SwiGLU, the gate) on the f32 router, and the
    bf16 output on the quantised one."""
    p, x = _c1_params(orc, fs=256, router_bits=router_bits)
    out1, idx1, w1 = orc.block_forward(p, x)
    p0 = dict(p)
    for k in ("shared_gate", "shared_up", "shared_down", "shared_gate_w", "shared_gate_q"):
        p0.pop(k, None)
    p0["fs"] = 0
    out0, idx0, w0 = orc.block_forward(p0, x)
    assert np.array_equal(idx0, idx1) and np.array_equal(w0, w1)
    if router_bits:
        out1, out0 = orc.bf16_to_f32(out1), orc.bf16_to_f32(out0)
    got = out1.astype(np.float64) - out0.astype(np.float64)
    xf = orc.bf16_to_f32(x).astype(np.float64)
    deq = lambda t: orc.bf16_to_f32(orc.dequantize(*t, 64, 4))[0].astype(np.float64)
    g = xf @ deq(p["shared_gate"]).T
    u = xf @ deq(p["shared_up"]).T
    ys = ((g / (1.0 + np.exp(-g))) * u) @ deq(p["shared_down"]).T
    if router_bits:
        gw = orc.dequantize(*p["shared_gate_q"], 64, 8, out_bf16=False)
        sl = xf @ gw.astype(np.float64)[0]
    else:
        sl = xf @ p["shared_gate_w"].astype(np.float64)[0]
    gate = 1.0 / (1.0 + np.exp(-sl))
    assert np.all((gate > 0.05) & (gate < 0.95)) and np.ptp(gate) > 0.3
    want = gate[:, None] * ys
    rms = np.sqrt(np.mean(want ** 2))
    # The bf16 roundings are unbiased noise: about 0.4% of the RMS on
    # average, a few percent at the worst of 8192 elements.  A bf16 out
    # (quantised router) adds up to one bf16 step of the routed part.
    err = np.abs(got - want)
    assert err.mean() <= 1e-2 * rms
    assert np.all(err <= 8e-2 * rms + (2.0 ** -7 * np.abs(out0) if router_bits else 0.0))
    # an ungated branch, or a constant gate of 1/2, is far outside
    assert np.abs(ys - want).mean() > 10 * 1e-2 * rms
    assert np.abs(0.5 * ys - want).mean() > 10 * 1e-2 * rms


# ------------------------------------------------------------ dispatch
def test_dispatch_is_stable_argsort(orc):
    rng = np.random.default_rng(7)
    for n, E in [(1, 1), (37, 4), (4096, 128), (20480, 512)]:
        ids = rng.integers(0, E, n).astype(np.int32)
        counts, offsets, srt, inv = orc.dispatch(ids, E)
        order = np.argsort(ids, kind="stable")
        assert np.array_equal(srt, order)
        assert np.array_equal(inv, np.argsort(order, kind="stable"))
        assert np.array_equal(counts, np.bincount(ids, minlength=E))
        assert offsets[0] == 0 and np.array_equal(np.diff(offsets), counts)
    with pytest.raises(ValueError):
        orc.dispatch(np.array([0, 4], np.int32), 4)


# ---------------------------------------------------------- gather_qmm
def _dense(orc, wq, sc, bi, bits):
    return orc.dequantize(wq, sc, bi, 64, bits, out_bf16=False).astype(np.float64)


@pytest.mark.parametrize("bits", [4, 8])
def test_gather_qmm_equals_gather_mm_of_dequant(orc, bits):
    """quantization.rs:344-421: gather_qmm == gather_mm(x, dequant(w)^T)
    for (lhs=(0,), rhs=(2,1)) and (x batch 5, lhs=(0,2), rhs=(2,1))."""
    rng = np.random.default_rng(8)
    M, N, K = 32, 64, 64
    wf = orc.f32_to_bf16(rng.standard_normal((3, N, K)).astype(np.float32))
    wq, sc, bi = orc.quantize(wf, 64, bits)
    wd = _dense(orc, wq, sc, bi, bits)
    for xb, lhs in [(1, [0]), (5, [0, 2])]:
        x = orc.f32_to_bf16(rng.standard_normal((xb, M, K)).astype(np.float32))
        rhs = [2, 1]
        lhs_use = lhs if len(lhs) == 2 else [0, 0]
        got = orc.bf16_to_f32(orc.gather_qmm(x, wq, sc, bi, rhs, lhs_use, bits=bits))
        xf = orc.bf16_to_f32(x).astype(np.float64)
        want = np.stack([xf[lhs_use[i]] @ wd[rhs[i]].T for i in range(2)])
        assert np.allclose(got, want, rtol=2 ** -7, atol=1e-3 * np.abs(want).max())


@pytest.mark.parametrize("bits", [4, 8])
def test_gather_qmm_tiled_is_gather_mm_of_bf16_dequant(orc, bits):
    """The tiled numerics are gather_mm(x, dequantize(w)^T) with the
    dequantised weights in bf16 (the array dtype), as the reference test
    states gather_qmm (quantization.rs:344-421): every product is exact in
    f32, so only the f32 accumulation separates it from an fp64 matmul of
    the bf16 dequantize output; the vector numerics keep f32 weights and do
    differ from it."""
    rng = np.random.default_rng(18)
    E, N, K, T = 3, 64, 256, 40
    wq, sc, bi = orc.quantize(orc.f32_to_bf16(0.02 * rng.standard_normal((E, N, K)).astype(np.float32)),
                              64, bits)
    wd16 = orc.bf16_to_f32(orc.dequantize(wq, sc, bi, 64, bits, out_bf16=True)).astype(np.float64)
    x = orc.f32_to_bf16(rng.standard_normal((T, 1, K)).astype(np.float32))
    rhs = rng.integers(0, E, T).astype(np.int32)
    xf = orc.bf16_to_f32(x).astype(np.float64)[:, 0]
    exact = np.stack([wd16[rhs[t]] @ xf[t] for t in range(T)])
    bound = np.stack([np.abs(wd16[rhs[t]]) @ np.abs(xf[t]) for t in range(T)])
    tiled = orc.bf16_to_f32(orc.gather_qmm(x, wq, sc, bi, rhs, bits=bits, tiled=True))[:, 0]
    # f32 accumulation error (K terms) plus the final bf16 rounding
    assert np.all(np.abs(tiled - exact) <= K * 2.0 ** -24 * bound + 2.0 ** -8 * np.abs(exact) + 1e-30)
    vec = orc.gather_qmm(x, wq, sc, bi, rhs, bits=bits, tiled=False)[:, 0]
    assert not np.array_equal(vec, orc.f32_to_bf16(tiled.astype(np.float32)))


def test_gather_qmm_broadcast_x_over_topk(orc):
    """x [T, 1, K] against indices [T, k]: out row (t, j) uses x[t]."""
    rng = np.random.default_rng(9)
    T, k, E, N, K = 6, 3, 5, 64, 128
    wq, sc, bi = orc.quantize(orc.f32_to_bf16(rng.standard_normal((E, N, K)).astype(np.float32)))
    x = orc.f32_to_bf16(rng.standard_normal((T, 1, K)).astype(np.float32))
    idx = rng.integers(0, E, (T, k)).astype(np.int32)
    got = orc.gather_qmm(x, wq, sc, bi, idx.reshape(-1))
    lhs = np.repeat(np.arange(T), k)
    assert np.array_equal(got, orc.gather_qmm(x, wq, sc, bi, idx.reshape(-1), lhs))


# -------------------------------------------------------------- swiglu
def test_swiglu_reference_values(orc):
    """activations.rs:341-351 inputs: silu(g) * u vs the manual formula."""
    g = np.array([1.0, -1.0, 0.5, 2.0], np.float32)
    u = np.array([1.0, 2.0, 3.0, 4.0], np.float32)
    got = orc.bf16_to_f32(orc.swiglu(orc.f32_to_bf16(g), orc.f32_to_bf16(u)))
    want = g / (1 + np.exp(-g.astype(np.float64))) * u
    assert np.allclose(got, want, rtol=3 * 2 ** -8)


# --------------------------------------------------------------- block
def _c1_params(orc, seed=0, K=2, E=8, fs=0, bits=4, bias=False, router_bits=0):
    rng = np.random.default_rng(seed)
    d, f = 512, 256

    def q(shape):
        w = orc.f32_to_bf16((rng.standard_normal(shape) * 0.02).astype(np.float32))
        return orc.quantize(w, 64, bits)

    p = dict(d=d, E=E, K=K, f=f, fs=fs, bits=bits, group_size=64,
             router_w=(rng.standard_normal((E, d)) * 0.02).astype(np.float32),
             router_b=(rng.standard_normal(E).astype(np.float32) if bias else None),
             gate=q((E, f, d)), up=q((E, f, d)), down=q((E, d, f)))
    if fs:
        p.update(shared_gate=q((1, fs, d)), shared_up=q((1, fs, d)), shared_down=q((1, d, fs)),
                 shared_gate_w=(rng.standard_normal((1, d)) * 0.02).astype(np.float32))
    if router_bits:
        # QuantizedLinear router and shared gate, quantised from bf16
        rq = lambda a: orc.quantize(orc.f32_to_bf16(a), 64, router_bits)
        p.update(router_w=None, router_b=None, router_bits=router_bits,
                 router_q=rq((rng.standard_normal((E, d)) * 0.05).astype(np.float32)))
        if fs:
            p.update(shared_gate_w=None,
                     shared_gate_q=rq((rng.standard_normal((1, d)) * 0.05).astype(np.float32)))
    x = orc.f32_to_bf16(rng.standard_normal((16, d)).astype(np.float32))
    return p, x


@pytest.mark.parametrize("fs,bias", [(0, False), (256, False), (0, True)])
def test_block_equals_sorted_composition(orc, fs, bias):
    """switch.rs:446-474: the sorted path (gather_sort -> gather_qmm ->
    swiglu -> gather_qmm -> scatter_unsort -> combine) and the block's
    per-(t, k) path give identical bits."""
    p, x = _c1_params(orc, fs=fs, bias=bias)
    out, idx, w = orc.block_forward(p, x)
    T, K, d, f = x.shape[0], p["K"], p["d"], p["f"]
    lg = orc.router_logits(x, p["router_w"])
    if bias:
        lg = (lg + p["router_b"]).astype(np.float32)
    idx2, w2 = orc.router_topk(lg, K)
    assert np.array_equal(idx, idx2) and np.array_equal(w, w2)
    _, _, order, inv = orc.dispatch(idx, p["E"])
    rows = order // K
    xs = x[rows][:, None, :]
    ids = idx.reshape(-1)[order]
    g = orc.gather_qmm(xs, *p["gate"], ids)
    u = orc.gather_qmm(xs, *p["up"], ids)
    a = orc.swiglu(g, u)
    y = orc.gather_qmm(a, *p["down"], ids)[inv].reshape(T, K, d)
    sy = sl = None
    if fs:
        x1 = x[:, None, :]
        zeros = np.zeros(T, np.int32)
        sa = orc.swiglu(orc.gather_qmm(x1, *p["shared_gate"], zeros),
                        orc.gather_qmm(x1, *p["shared_up"], zeros))
        sy = orc.gather_qmm(sa, *p["shared_down"], zeros).reshape(T, d)
        sl = orc.router_logits(x, p["shared_gate_w"])[:, 0]
    assert np.array_equal(out, orc.combine(y, w, sy, sl))


@pytest.mark.parametrize("fs", [0, 256])
def test_block_quantised_router_equals_composition(orc, fs):
    """With an 8-bit QuantizedLinear router and shared gate the block is
    bf16 throughout: router_logits_q -> router_topk_bf16 -> the sorted
    expert path -> combine_bf16, bit for bit."""
    p, x = _c1_params(orc, fs=fs, router_bits=8)
    out, idx, w = orc.block_forward(p, x)
    assert out.dtype == np.uint16
    T, K, d = x.shape[0], p["K"], p["d"]
    lg = orc.router_logits_q(x, *p["router_q"], 8)
    idx2, w2 = orc.router_topk_bf16(lg, K)
    assert np.array_equal(idx, idx2) and np.array_equal(w, w2)
    _, _, order, inv = orc.dispatch(idx, p["E"])
    xs = x[order // K][:, None, :]
    ids = idx.reshape(-1)[order]
    a = orc.swiglu(orc.gather_qmm(xs, *p["gate"], ids), orc.gather_qmm(xs, *p["up"], ids))
    y = orc.gather_qmm(a, *p["down"], ids)[inv].reshape(T, K, d)
    sy = sl = None
    if fs:
        x1 = x[:, None, :]
        zeros = np.zeros(T, np.int32)
        sa = orc.swiglu(orc.gather_qmm(x1, *p["shared_gate"], zeros),
                        orc.gather_qmm(x1, *p["shared_up"], zeros))
        sy = orc.gather_qmm(sa, *p["shared_down"], zeros).reshape(T, d)
        sl = orc.router_logits_q(x, *p["shared_gate_q"], 8)[:, 0]
    assert np.array_equal(out, orc.combine_bf16(y, w, sy, sl))


def test_block_top1_is_single_expert(orc):
    p, x = _c1_params(orc, K=1)
    out, idx, w = orc.block_forward(p, x)
    assert np.all(w == 1.0)
    e = idx[:, 0]
    g = orc.gather_qmm(x[:, None, :], *p["gate"], e)
    u = orc.gather_qmm(x[:, None, :], *p["up"], e)
    y = orc.gather_qmm(orc.swiglu(g, u), *p["down"], e).reshape(16, -1)
    assert np.array_equal(out, orc.bf16_to_f32(y))


def test_block_zero_input(orc):
    p, x = _c1_params(orc)
    out, idx, w = orc.block_forward(p, np.zeros_like(x))
    assert np.all(idx == [0, 1]) and np.allclose(w, 0.5)
    # biases of the quantised weights make gate(0) = 0 exactly (x = 0)
    assert np.all(out == 0.0)


def test_combine_linear_in_weights(orc):
    rng = np.random.default_rng(10)
    y = orc.f32_to_bf16(rng.standard_normal((4, 3, 64)).astype(np.float32))
    w1 = rng.random((4, 3)).astype(np.float32)
    w2 = rng.random((4, 3)).astype(np.float32)
    lhs = orc.combine(y, w1 + w2)
    rhs = orc.combine(y, w1) + orc.combine(y, w2)
    assert np.allclose(lhs, rhs, rtol=1e-5, atol=1e-6)


# ----------------------------------------------- gemma4: GeGLU, router
def test_geglu_closed_forms_and_fp64_bound(orc):
    """gelu_approx(g) * u (activations.rs:223-259): large positive g pass
    through (tanh -> 1), large negative g give 0 (tanh -> -1), g = 0 gives
    0; elsewhere within a few bf16 roundings of the fp64 tanh-GELU."""
    bf = lambda a: orc.f32_to_bf16(np.asarray(a, np.float32))  # noqa: E731
    f = lambda h: orc.bf16_to_f32(h).astype(np.float64)  # noqa: E731
    big = np.array([4.0, 5.5, 8.0, 17.0, 96.0], np.float32)
    assert np.array_equal(orc.geglu(bf(big), bf(np.ones_like(big))), bf(big))
    neg = np.array([-6.0, -9.0, -40.0], np.float32)
    assert np.all(f(orc.geglu(bf(neg), bf(np.ones_like(neg)))) == 0.0)
    assert f(orc.geglu(bf([0.0]), bf([3.0])))[0] == 0.0
    rng = np.random.default_rng(50)
    g = bf(rng.standard_normal(4096) * 2)
    u = bf(rng.standard_normal(4096))
    gd, ud = f(g), f(u)
    exact = 0.5 * gd * (1 + np.tanh(np.sqrt(2 / np.pi) * (gd + 0.044715 * gd ** 3))) * ud
    got = f(orc.geglu(g, u))
    assert np.all(np.abs(got - exact) <= 2.0 ** -5 * (np.abs(gd) + 0.05) * np.abs(ud))


def _geglu_torch_bf16(g, u):
    """gelu_approximate_in_dtype(g) * u op for op as activations.rs:246-259
    builds it, on torch's CPU bfloat16 arithmetic (every op computed in f32
    and rounded to bf16, the constants cast to bf16 first): an
    implementation of the same op graph independent of the oracle's C."""
    import math

    import torch
    bf = torch.bfloat16
    c = lambda v: torch.tensor(v, dtype=torch.float32).to(bf)  # noqa: E731
    x = torch.from_numpy(np.asarray(g, np.float32)).to(bf)
    uu = torch.from_numpy(np.asarray(u, np.float32)).to(bf)
    half, one = c(0.5), c(1.0)
    s2p, k = c(math.sqrt(2.0 / math.pi)), c(0.044715)
    x3 = x * x * x
    t = torch.tanh(s2p * (x + k * x3))
    return ((half * x * (one + t)) * uu).float().numpy()


def test_geglu_bf16_chain_pinned(orc):
    """The tanh-approximate GELU in bf16 (activations.rs:246-259), pinned
    where the erf GELU and the approximation part: on every bf16 g with
    |g| <= 6 (and random u) the oracle equals the same op graph on torch's
    bf16 arithmetic bit for bit.  Hand-worked: g = -3, u = 1 gives
    x^3 = -27, k*x^3 = bf16(0.044677734375 * -27) = -1.203125,
    inner = bf16(-4.203125) = -4.1875 (tie to even),
    bf16(0.796875 * -4.1875) = -3.34375, bf16(tanh) = -0.99609375,
    1 + t = 2^-8, out = -1.5 * 2^-8 = -0.005859375 -- where the fp64
    tanh form gives -0.00364 and the erf GELU -0.00405."""
    f = lambda h: orc.bf16_to_f32(h).astype(np.float64)  # noqa: E731
    bf = lambda a: orc.f32_to_bf16(np.asarray(a, np.float32))  # noqa: E731
    assert f(orc.geglu(bf([-3.0]), bf([1.0])))[0] == -0.005859375
    allb = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    gv = orc.bf16_to_f32(allb)
    g = allb[np.isfinite(gv) & (np.abs(gv) <= 6.0)]
    rng = np.random.default_rng(53)
    for u in (np.ones(g.size, np.float32), rng.standard_normal(g.size).astype(np.float32)):
        ub = bf(u)
        want = _geglu_torch_bf16(orc.bf16_to_f32(g), orc.bf16_to_f32(ub))
        got = orc.bf16_to_f32(orc.geglu(g, ub))
        assert np.array_equal(got, want)
    # the test tells the two GELUs apart: on [-4, -2.5] the erf form moves
    # most outputs by many bf16 steps
    tail = g[(orc.bf16_to_f32(g) >= -4.0) & (orc.bf16_to_f32(g) <= -2.5)]
    import math
    gt = orc.bf16_to_f32(tail).astype(np.float64)
    erf = bf(0.5 * gt * (1 + np.array([math.erf(v / math.sqrt(2)) for v in gt])))
    assert np.mean(orc.geglu(tail, bf(np.ones(tail.size))) != erf) > 0.5


def test_rms_norm_eps_pinned(orc):
    """fast::rms_norm's eps (normalization.rs:272-276): a row where eps
    dominates the mean square (x = 2^-10, mean(x^2) = 2^-20, eps = 1e-3)
    gives w * x / sqrt(mean(x^2) + eps) = 0.03087 within one bf16 rounding
    (without eps it would be 1.0); and the reference's own known answer
    (fast.rs:726-741: [1, 2, 3, 4] with eps 1e-5, no weight, against
    x * rsqrt(mean(x^2) + eps)) with a unit weight, within one bf16
    rounding."""
    d = 512
    x = orc.f32_to_bf16(np.full((1, d), 2.0 ** -10, np.float32))
    w = orc.f32_to_bf16(np.ones(d, np.float32))
    got = orc.bf16_to_f32(orc.rms_norm(x, w, 1e-3)).astype(np.float64)
    want = 2.0 ** -10 / np.sqrt(2.0 ** -20 + float(np.float32(1e-3)))
    assert np.all(np.abs(got - want) <= 2.0 ** -8 * want)
    assert np.all(np.abs(got - 1.0) > 0.5)
    a = np.array([[1.0, 2.0, 3.0, 4.0]], np.float32)
    got = orc.bf16_to_f32(orc.rms_norm(orc.f32_to_bf16(a), orc.f32_to_bf16(np.ones(4, np.float32)),
                                       1e-5)).astype(np.float64)
    want = a / np.sqrt((a.astype(np.float64) ** 2).mean() + 1e-5)
    assert np.all(np.abs(got - want) <= 2.0 ** -8 * np.abs(want))


def test_rms_norm_exact_and_fp64_bound(orc):
    """fast::rms_norm: a constant row 2 with eps 0 normalises to 1, so the
    output is the weight exactly; elsewhere within two bf16 roundings of
    w * x / sqrt(mean(x^2) + eps)."""
    rng = np.random.default_rng(51)
    d = 512
    w = orc.f32_to_bf16((rng.random(d) + 0.5).astype(np.float32))
    x = orc.f32_to_bf16(np.full((1, d), 2.0, np.float32))
    assert np.array_equal(orc.rms_norm(x, w, 0.0)[0], w)
    x = orc.f32_to_bf16(rng.standard_normal((7, d)).astype(np.float32))
    got = orc.bf16_to_f32(orc.rms_norm(x, w, 1e-6)).astype(np.float64)
    xd = orc.bf16_to_f32(x).astype(np.float64)
    exact = orc.bf16_to_f32(w).astype(np.float64) * xd / np.sqrt(
        (xd ** 2).mean(1, keepdims=True) + 1e-6)
    assert np.all(np.abs(got - exact) <= 2.0 ** -7 * np.abs(exact) + 1e-30)


@pytest.mark.parametrize("bits", [0, 8])
def test_gemma_router(orc, bits):
    """gemma4 Router::forward (text.rs:621-665): top-K = full sort of the
    bf16 scores (ties to the lower id); weights = bf16 softmax of the K
    selected scores times per_expert_scale: within bf16 roundings of the
    fp64 softmax, and exactly linear in per_expert_scale (x2 is exact)."""
    rng = np.random.default_rng(52 + bits)
    T, d, E, K = 24, 512, 16, 4
    x = orc.f32_to_bf16(rng.standard_normal((T, d)).astype(np.float32))
    nw = orc.f32_to_bf16(np.full(d, d ** -0.5, np.float32))
    projf = orc.f32_to_bf16(rng.standard_normal((E, d)).astype(np.float32))
    proj = orc.quantize(projf, 64, 8) if bits else projf
    pes = orc.f32_to_bf16((rng.random(E) + 0.5).astype(np.float32))
    idx, w = orc.gemma_router(x, nw, 1e-6, proj, pes, K, bits=bits)
    normed = orc.rms_norm(x, nw, 1e-6)
    if bits:
        sc = orc.router_logits_q(normed, *proj, 8)
    else:
        sc = orc.bf16_to_f32(orc.f32_to_bf16(orc.router_logits(normed, orc.bf16_to_f32(projf))))
    for t in range(T):
        order = sorted(range(E), key=lambda e: (-float(sc[t, e]), e))
        assert list(idx[t]) == order[:K]
    s = np.take_along_axis(sc, idx, 1).astype(np.float64)
    p = np.exp(s - s.max(1, keepdims=True))
    p /= p.sum(1, keepdims=True)
    exact = p * orc.bf16_to_f32(pes)[idx]
    got = orc.bf16_to_f32(w).astype(np.float64)
    assert np.all(np.abs(got - exact) <= 2.0 ** -6 * exact + 1e-6)
    _, w2 = orc.gemma_router(x, nw, 1e-6, proj, orc.f32_to_bf16(2 * orc.bf16_to_f32(pes)), K,
                             bits=bits)
    assert np.array_equal(orc.bf16_to_f32(w2), 2 * orc.bf16_to_f32(w))


@pytest.mark.parametrize("act", [0, 1])
def test_packed_switch_glu_equals_split_composition(orc, act):
    """PackedSwitchFfn (switch.rs:290-335): gate_up [E, 2H, d] is gate and up
    stacked along the output rows; the forward equals gather_qmm of each
    half, the activation (SwiGLU / GeGLU), the down gather_qmm and the
    combine, bit for bit, with f32 or bf16 routing weights."""
    rng = np.random.default_rng(53 + act)
    T, d, H, E, K = 12, 512, 256, 8, 2

    def q(shape):
        return orc.quantize(orc.f32_to_bf16((rng.standard_normal(shape) * 0.02).astype(np.float32)),
                            64, 4)
    gate, up, down = q((E, H, d)), q((E, H, d)), q((E, d, H))
    gu = tuple(np.concatenate([a, b], axis=1) for a, b in zip(gate, up))
    x = orc.f32_to_bf16(rng.standard_normal((T, d)).astype(np.float32))
    idx = np.stack([rng.permutation(E)[:K] for _ in range(T)]).astype(np.int32)
    wf = rng.random((T, K)).astype(np.float32)
    wb = orc.bf16_to_f32(orc.f32_to_bf16(wf))
    flat = idx.reshape(-1)
    xs = x[np.repeat(np.arange(T), K)][:, None, :]
    g = orc.gather_qmm(xs, *gate, flat)
    u = orc.gather_qmm(xs, *up, flat)
    a = orc.geglu(g, u) if act else orc.swiglu(g, u)
    y = orc.gather_qmm(a, *down, flat).reshape(T, K, d)
    out_f, y_got = orc.packed_switch_glu(x, gu, down, idx, wf, act=act, w_bf16=False, with_y=True)
    assert np.array_equal(y_got, y)
    assert np.array_equal(out_f, orc.combine(y, wf))
    out_b = orc.packed_switch_glu(x, gu, down, idx, wb, act=act, w_bf16=True)
    assert np.array_equal(out_b, orc.combine_bf16(y, wb))


# ------------------------------------------------- dense gather_mm (bf16)
def test_gather_mm_reference_example(orc):
    """arithmetic.rs:1565-1575: a = ones [5, 32, 32], b = ones [3, 32, 32],
    lhs (0, 2), rhs (2, 1) -> [2, 32, 32], every entry 32."""
    one = orc.f32_to_bf16(np.ones(1, np.float32))[0]
    a = np.full((5, 32, 32), one, np.uint16)
    b = np.full((3, 32, 32), one, np.uint16)
    out = orc.gather_mm(a, b, [2, 1], [0, 2])
    assert out.shape == (2, 32, 32)
    assert np.all(orc.bf16_to_f32(out) == 32.0)


def test_gather_mm_fp64_bound_and_indices(orc):
    """f32 accumulation of exact bf16 products: within K * 2^-24 * |x||w| of
    the fp64 matmul, then one bf16 rounding; lhs indices and the x broadcast
    over the trailing index axis pick the same rows."""
    rng = np.random.default_rng(31)
    E, N, K, T, k = 5, 96, 320, 7, 3
    w = orc.f32_to_bf16(rng.standard_normal((E, N, K)).astype(np.float32))
    x = orc.f32_to_bf16(rng.standard_normal((T, 1, K)).astype(np.float32))
    idx = rng.integers(0, E, (T, k)).astype(np.int32).reshape(-1)
    got = orc.bf16_to_f32(orc.gather_mm(x, w, idx))[:, 0].astype(np.float64)
    wf = orc.bf16_to_f32(w).astype(np.float64)
    xf = orc.bf16_to_f32(x).astype(np.float64)[:, 0]
    rows = np.repeat(np.arange(T), k)
    exact = np.stack([wf[idx[i]] @ xf[rows[i]] for i in range(T * k)])
    bound = np.stack([np.abs(wf[idx[i]]) @ np.abs(xf[rows[i]]) for i in range(T * k)])
    assert np.all(np.abs(got - exact) <= K * 2.0 ** -24 * bound + 2.0 ** -8 * np.abs(exact))
    assert np.array_equal(orc.gather_mm(x, w, idx), orc.gather_mm(x, w, idx, rows))


def test_gather_mm_is_tiled_gather_qmm_of_dequant(orc):
    """quantization.rs:344-421 states gather_qmm(x, w) == gather_mm(x,
    dequantize(w)^T): at 4 bits the oracle's tiled gather_qmm and its
    gather_mm over the bf16 dequantised weights sum the same products in the
    same order, so they agree bit for bit."""
    rng = np.random.default_rng(32)
    E, N, K, T = 4, 64, 256, 24
    wq, sc, bi = orc.quantize(orc.f32_to_bf16(0.02 * rng.standard_normal((E, N, K)).astype(np.float32)),
                              64, 4)
    wd = orc.dequantize(wq, sc, bi, 64, 4, out_bf16=True).reshape(E, N, K)
    x = orc.f32_to_bf16(rng.standard_normal((T, 1, K)).astype(np.float32))
    rhs = rng.integers(0, E, T).astype(np.int32)
    assert np.array_equal(orc.gather_qmm(x, wq, sc, bi, rhs, bits=4, tiled=True),
                          orc.gather_mm(x, wd, rhs))


def _dequant_params(orc, p):
    """The block parameters with every 4-bit expert bank replaced by its bf16
    dequantisation (dense SwitchLinear / Linear weights)."""
    d = dict(p, bits=16)
    for k in ("gate", "up", "down", "shared_gate", "shared_up", "shared_down"):
        if p.get(k) is not None:
            wq, sc, bi = p[k]
            E, N = wq.shape[0], wq.shape[1]
            K = wq.shape[2] * 32 // p["bits"]
            d[k] = (orc.dequantize(wq, sc, bi, 64, p["bits"], out_bf16=True).reshape(E, N, K),
                    None, None)
    return d


@pytest.mark.parametrize("fs", [0, 256])
def test_block_dense_experts_equal_tiled_4bit_block(orc, fs):
    """A block with dense bf16 experts (gather_mm) equals, bit for bit, the
    4-bit block whose weights dequantise to them, on the tiled numerics
    (gather_qmm == gather_mm(dequantize(w)), quantization.rs:344-421)."""
    p, x = _c1_params(orc, fs=fs)
    ref, ridx, rw = orc.block_forward(p, x, tiled=(True, True))
    got, gidx, gw = orc.block_forward(_dequant_params(orc, p), x)
    assert np.array_equal(gidx, ridx) and np.array_equal(gw, rw)
    assert np.array_equal(got, ref)


def _exact_q8(orc, rng, shape):
    """8-bit codes with scale 2^-7 and bias -1: every dequantised weight
    code/128 - 1 is exact in f32 and in bf16.  Returns the QuantizedLinear
    (wq, scales, biases) and the same weights as bf16 bits."""
    rows, d = shape
    codes = rng.integers(0, 256, (rows, d)).astype(np.uint32)
    c4 = codes.reshape(rows, d // 4, 4)
    wq = c4[..., 0] | (c4[..., 1] << 8) | (c4[..., 2] << 16) | (c4[..., 3] << 24)
    sc = np.full((rows, d // 64), orc.f32_to_bf16(np.float32(2.0 ** -7)), np.uint16)
    bi = np.full((rows, d // 64), orc.f32_to_bf16(np.float32(-1.0)), np.uint16)
    wd = orc.f32_to_bf16((codes.astype(np.float32) / 128.0 - 1.0).astype(np.float32))
    return (wq.astype(np.uint32), sc, bi), wd


def test_bf16_linear_router_equals_exact_8bit_router(orc):
    """A bf16 Linear router (bits 16) computes what the 8-bit
    QuantizedLinear router computes when its codes dequantise exactly to the
    bf16 weights: the same logits, routing and block output, bit for bit."""
    rng = np.random.default_rng(33)
    p, x = _c1_params(orc, fs=256, router_bits=8)
    rq, rd = _exact_q8(orc, rng, (p["E"], p["d"]))
    sq, sd = _exact_q8(orc, rng, (1, p["d"]))
    # scale the router input so the logits stay O(1)
    x = orc.f32_to_bf16((orc.bf16_to_f32(x) * 0.02).astype(np.float32))
    lq = orc.router_logits_q(x, *rq, 8)
    ld = orc.router_logits_q(x, rd, None, None, 16)
    assert np.array_equal(lq, ld)
    p8 = dict(p, router_q=rq, shared_gate_q=sq, router_bits=8)
    p16 = dict(p, router_q=(rd, None, None), shared_gate_q=(sd, None, None), router_bits=16)
    o8, i8, w8 = orc.block_forward(p8, x)
    o16, i16, w16 = orc.block_forward(p16, x)
    assert np.array_equal(i8, i16) and np.array_equal(w8, w16) and np.array_equal(o8, o16)
    # fp64 bound on the dense logits themselves
    xf = orc.bf16_to_f32(x).astype(np.float64)
    wf = orc.bf16_to_f32(rd).astype(np.float64)
    exact = xf @ wf.T
    bound = np.abs(xf) @ np.abs(wf).T
    assert np.all(np.abs(ld - exact) <= p["d"] * 2.0 ** -24 * bound + 2.0 ** -8 * np.abs(exact))


def test_packed_switch_glu_dense_equals_split_composition(orc):
    """PackedSwitchFfn over a dense [E, 2H, d] gate_up (SwitchLinear) is the
    two gather_mm halves, the activation, the down gather_mm and the
    combine."""
    rng = np.random.default_rng(34)
    E, d, H, T, K = 6, 256, 128, 9, 2
    gu = orc.f32_to_bf16((0.05 * rng.standard_normal((E, 2 * H, d))).astype(np.float32))
    dn = orc.f32_to_bf16((0.05 * rng.standard_normal((E, d, H))).astype(np.float32))
    x = orc.f32_to_bf16(rng.standard_normal((T, d)).astype(np.float32))
    idx = np.stack([rng.permutation(E)[:K] for _ in range(T)]).astype(np.int32)
    w = rng.random((T, K)).astype(np.float32)
    for act, fn in ((1, orc.geglu), (0, orc.swiglu)):
        out = orc.packed_switch_glu(x, (gu, None, None), (dn, None, None), idx, w, act=act,
                                    w_bf16=False)
        ids = idx.reshape(-1)
        xs = np.repeat(x, K, axis=0)[:, None, :]
        g = orc.gather_mm(xs, np.ascontiguousarray(gu[:, :H]), ids)
        u = orc.gather_mm(xs, np.ascontiguousarray(gu[:, H:]), ids)
        y = orc.gather_mm(fn(g, u), dn, ids).reshape(T, K, d)
        assert np.array_equal(out, orc.combine(y, w))


# ------------------------------------------- the decoder layer's MoE half
@pytest.mark.parametrize("router_bits", [0, 8])
def test_block_residual_zero_norm_is_identity(orc, router_bits):
    """layer.rs:134-138 with a zero norm weight: the block sees zero rows,
    whose expert outputs are zero (no biases), so out = h exactly -- f32(h)
    with the f32 router, h itself in the bf16 chain."""
    p, h = _c1_params(orc, fs=256, router_bits=router_bits)
    out, _, _ = orc.block_forward_residual(p, np.zeros(p["d"], np.uint16), 1e-6, h)
    if router_bits:
        assert out.dtype == np.uint16 and np.array_equal(out, h)
    else:
        assert np.array_equal(out, orc.bf16_to_f32(h))


@pytest.mark.parametrize("router_bits", [0, 8])
def test_block_residual_equals_norm_block_add(orc, router_bits):
    """The fused tail equals its op sequence: post_attention_layernorm
    (fast::rms_norm), the block, and the add in the block output's dtype
    (bf16 + f32 promotes; bf16 + bf16 rounds to bf16)."""
    rng = np.random.default_rng(70)
    p, h = _c1_params(orc, fs=256, router_bits=router_bits)
    nw = orc.f32_to_bf16((1.0 + 0.1 * rng.standard_normal(p["d"])).astype(np.float32))
    out, idx, w = orc.block_forward_residual(p, nw, 1e-6, h)
    m, idx2, w2 = orc.block_forward(p, orc.rms_norm(h, nw, 1e-6))
    assert np.array_equal(idx, idx2) and np.array_equal(w, w2)
    hf = orc.bf16_to_f32(h)
    if router_bits:
        want = orc.f32_to_bf16((hf + orc.bf16_to_f32(m)).astype(np.float32))
    else:
        want = (hf + m).astype(np.float32)
    assert np.array_equal(out, want)
