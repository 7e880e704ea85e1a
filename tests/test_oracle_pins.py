"""Pins of the CPU oracle (oracle/bq_oracle.c) against what mathematics or an
independent library fixes, so that a dropped term, a wrong sign or index, or a
transposed operand in the restatement fails here.  The reference ships no
golden vectors for this path (its tests never call the butterquant GEMMs), so
these pins plus the committed fixtures in tests/golden/ are the parity anchor.

Pin map (oracle function -> pins):
  fwht_block/row      unit-vector KAT (exact Sylvester signs x c_B), f64 matrix
                      closed form, involution, Parseval, scale-constant KATs
  quant_segment       tie-to-even KATs, zero segment, amax -> +-127
  f32_to_bf16         torch's independent RNE conversion
  rms_reduce_row      f64 sum of squares
  prepare_norm_act.   f64 pipeline (codes within 1, scale rel 1e-5)
  prepare_block_act.  f64 pipeline
  pack_and_colsum     hand-derived byte positions, bijection, int64 row sums
  gemm per-row/block  int64 brute force + f64 epilogue closed forms; VNNI
                      (u8, colsum) form == signed form
  exp/tanh/gelu fast  numpy exp/tanh/exact GELU within the stated error
  gelu_gate_up        up = 1 -> bf16(gelu(gate)); gate = 10 -> 10 * up;
                      gate = 0 -> 0; exact tanh-GELU product within bf16
  route top-k/softmax numpy stable argsort; weights sum to 1
  build_schedule      python stable sort of (expert, token, k)
  moe phase1/phase2   f64 closed forms over the unpacked weights
  router logits       f64 projection; one-hot rows (element order, scaling)
  exp_f32/log_f32     libm; SplitMix64 published outputs; Gumbel moments/CDF
  head_logit_row      exact integers at unit scales; f64 per-block chain
  flash_sample        numpy lexsort top-n, argmax, f64 logsumexp; filters
  embed_lookup        one-hot FWHT closed form, f64 rotation, shard zeros
"""
import ctypes as C
import math

import numpy as np
import pytest

BLOCKS = [16, 32, 64, 128, 256, 512]


def hadamard(b):
    i = np.arange(b)
    pc = np.vectorize(lambda v: bin(v).count("1"))(i[:, None] & i[None, :])
    return np.where(pc % 2 == 0, 1.0, -1.0)


@pytest.mark.parametrize("B", BLOCKS)
def test_fwht_unit_vector_kat(O, B):
    c = np.float32(O.fwht_scale(B))
    H = hadamard(B)
    for j in [0, 1, B // 2 - 1, B - 1, 5 % B]:
        e = np.zeros((1, B), np.float32)
        e[0, j] = 1.0
        y = O.fwht_rows(e, B)[0]
        np.testing.assert_array_equal(y, (H[:, j] * c).astype(np.float32))


def test_fwht_scale_constants(O):
    assert O.fwht_scale(16) == 0.25
    assert O.fwht_scale(64) == 0.125
    assert O.fwht_scale(256) == 0.0625
    for b in (32, 128, 512):
        assert O.fwht_scale(b) == float(np.float32(1.0 / float(np.sqrt(np.float32(b)))))


@pytest.mark.parametrize("B", BLOCKS)
def test_fwht_closed_form_involution_parseval(O, B):
    rng = np.random.default_rng(B)
    x = rng.standard_normal((3, 2 * B)).astype(np.float32)
    y = O.fwht_rows(x, B)
    H = hadamard(B) / math.sqrt(B)
    ref = np.concatenate([x[:, :B] @ H.T, x[:, B:] @ H.T], axis=1)
    assert np.abs(y - ref).max() <= 1e-5 * np.abs(ref).max() * math.log2(B)
    z = O.fwht_rows(y, B)
    assert np.abs(z - x).max() <= 1e-5 * np.abs(x).max() * math.log2(B)
    np.testing.assert_allclose(np.linalg.norm(y[:, :B], axis=1),
                               np.linalg.norm(x[:, :B], axis=1), rtol=1e-5)


def test_fwht_rejects_bad_block(O):
    with pytest.raises(ValueError):
        O.fwht_rows(np.zeros((1, 48), np.float32), 48)
    with pytest.raises(ValueError):
        O.fwht_rows(np.zeros((1, 96), np.float32), 64)


def test_quant_kats(O):
    q, s = O.quant_segment(np.array([127, 2.5, 3.5, -2.5, -0.5, 0.5, 1.5], np.float32), False)
    np.testing.assert_array_equal(q, [127, 2, 4, -2, 0, 0, 2])
    assert s == 127.0
    q, s = O.quant_segment(np.zeros(64, np.float32), True)
    assert (q == 0).all() and s == 0.0
    x = np.array([0.5, -2.0, 1.0, 0.25], np.float32)
    q, s = O.quant_segment(x, True)
    assert s == np.float32(2.0) / np.float32(127.0)
    np.testing.assert_array_equal(q, [32, -127, 64, 16])  # 31.75 -> 32, 63.5 -> 64 (even)


def test_quant_random_matches_numpy(O):
    rng = np.random.default_rng(7)
    x = rng.standard_normal(1000).astype(np.float32)
    q, s = O.quant_segment(x, False)
    amax = np.abs(x).max()
    inv = np.float32(127.0) / amax
    ref = np.clip(np.rint(x * inv), -128, 127).astype(np.int8)
    np.testing.assert_array_equal(q, ref)
    assert s == amax and np.abs(q).max() == 127


def test_bf16_rne_matches_torch(O):
    import torch
    rng = np.random.default_rng(1)
    x = np.concatenate([rng.standard_normal(4096).astype(np.float32) * 10.0 ** rng.integers(-8, 8, 4096),
                        np.array([1.0 + 2 ** -8, 1.0 + 3 * 2 ** -8, -1.0 - 2 ** -8, 0.0, -0.0,
                                  3.0e38, 1e-40], np.float32)]).astype(np.float32)
    mine = O.f32_to_bf16(x)
    ref = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    np.testing.assert_array_equal(mine, ref)
    c = np.array([O.lib().bqo_f32_to_bf16(float(v)) for v in x[:256]], np.uint16)
    np.testing.assert_array_equal(c, mine[:256])


@pytest.mark.parametrize("H", [2816, 4096, 2112, 128])
def test_rms_reduce_row_f64(O, H):
    x = O.synth_normal_bf16(3, 1.0, (H,))
    ss = O.rms_reduce_row(x)
    ref = float(np.sum(O.bf16_to_f32(x).astype(np.float64) ** 2))
    assert abs(ss - ref) <= 1e-5 * ref


@pytest.mark.parametrize("H,B", [(2816, 128), (4096, 128), (512, 64)])
def test_norm_quant_f64_pipeline(O, H, B):
    x = O.synth_normal_bf16(11, 1.0, (4, H))
    g = O.f32_to_bf16(np.linspace(0.5, 1.5, H).astype(np.float32))
    q, sa = O.norm_quant(x, g, B)
    sqrt_n, n_eps = O.norm_consts(H)
    xf = O.bf16_to_f32(x).astype(np.float64)
    inv = sqrt_n / np.sqrt((xf ** 2).sum(1, keepdims=True) + n_eps)
    w = xf * inv * O.bf16_to_f32(g)
    Hm = hadamard(B) / math.sqrt(B)
    w = (w.reshape(4, H // B, B) @ Hm.T).reshape(4, H)
    amax = np.abs(w).max(1)
    np.testing.assert_allclose(sa, amax, rtol=1e-5)
    ref = np.clip(np.rint(w * 127.0 / amax[:, None]), -128, 127)
    d = np.abs(q.astype(np.int64) - ref)
    assert d.max() <= 1 and (d == 0).mean() > 0.99


def test_block_quant_f64_pipeline(O):
    x = O.synth_normal_bf16(12, 1.0, (5, 704))
    q, sa = O.block_quant(x, 64, True)
    xf = O.bf16_to_f32(x).astype(np.float64).reshape(5, 11, 64) @ (hadamard(64) / 8.0).T
    amax = np.abs(xf).max(2)
    np.testing.assert_allclose(sa, amax, rtol=1e-5)
    ref = np.clip(np.rint(xf * 127.0 / amax[:, :, None]), -128, 127).reshape(5, 704)
    d = np.abs(q.astype(np.int64) - ref)
    assert d.max() <= 1 and (d == 0).mean() > 0.99
    # o_proj path: block = head_dim, no runtime FWHT (gemma_4_moe_bq.mojo:515-517)
    x2 = O.synth_normal_bf16(13, 1.0, (3, 1024))
    q2, sa2 = O.block_quant(x2, 256, False)
    x2f = O.bf16_to_f32(x2).astype(np.float64).reshape(3, 4, 256)
    np.testing.assert_array_equal(sa2, np.abs(x2f).max(2).astype(np.float32))
    ref2 = np.clip(np.rint(x2f * 127.0 / np.abs(x2f).max(2, keepdims=True)), -128, 127)
    assert np.abs(q2.astype(np.int64) - ref2.reshape(3, 1024)).max() <= 1
    with pytest.raises(ValueError):
        O.block_quant(x, 256, False)  # 704 is not a multiple of 256
    with pytest.raises(ValueError):
        O.block_quant(x, 48, True)


def test_pack_positions_and_bijection(O):
    rows, cols = 64, 128
    w = (np.arange(rows * cols) % 251 - 125).astype(np.int8).reshape(rows, cols)
    p, cs = O.pack_and_colsum(w)
    # a 32x64 tile is two 16-row halves; each half is the 16x16 dword transpose
    np.testing.assert_array_equal(p[0:4], w[0, 0:4])
    np.testing.assert_array_equal(p[4:8], w[1, 0:4])
    np.testing.assert_array_equal(p[60:64], w[15, 0:4])
    np.testing.assert_array_equal(p[64:68], w[0, 4:8])
    np.testing.assert_array_equal(p[1024:1028], w[16, 0:4])
    np.testing.assert_array_equal(p[2048:2052], w[0, 64:68])
    np.testing.assert_array_equal(p[32 * cols:32 * cols + 4], w[32, 0:4])
    off = O.vnni_offsets(rows, cols)
    assert np.unique(off).size == rows * cols and off.max() == rows * cols - 1
    np.testing.assert_array_equal(p[off], w)
    np.testing.assert_array_equal(cs, w.astype(np.int64).sum(1).astype(np.float32))
    p2, cs2 = O.pack_and_colsum(w, 64, False)
    np.testing.assert_array_equal(cs2.reshape(2, rows),
                                  w.astype(np.int64).reshape(rows, 2, 64).sum(2).T)
    with pytest.raises(ValueError):
        O.pack_and_colsum(w[:48])


def _quantized_linear(O, N, K, B, seed=0):
    wf = O.bf16_to_f32(O.synth_normal_bf16(seed, 0.02, (N, K)))
    q, s = O.rotate_and_quant(wf, B)
    return q, s


def test_rotate_and_quant_f64(O):
    wf = O.bf16_to_f32(O.synth_normal_bf16(0, 0.02, (32, 256)))
    q, s = O.rotate_and_quant(wf, 128)
    rot = (wf.astype(np.float64).reshape(32, 2, 128) @ (hadamard(128) / math.sqrt(128)).T).reshape(32, 256)
    np.testing.assert_allclose(s, np.abs(rot).max(1) / 127.0, rtol=1e-5)
    d = np.abs(q - np.clip(np.rint(rot / (np.abs(rot).max(1, keepdims=True) / 127.0)), -128, 127))
    assert d.max() <= 1
    qb, sb = O.rotate_and_quant(wf, 64, per_block=True)
    assert sb.shape == (32, 4)


@pytest.mark.parametrize("M", [1, 5])
def test_linear_closed_form(O, M):
    N, K = 64, 256
    q, s = _quantized_linear(O, N, K, 128)
    p, cs = O.pack_and_colsum(q)
    x = O.synth_normal_bf16(1, 1.0, (M, K))
    xq, sa = O.norm_quant(x, np.full(K, 0x3F80, np.uint16))
    ob, of = O.linear(xq, sa, p, s, cs, N)
    acc = xq.astype(np.int64) @ q.astype(np.int64).T
    np.testing.assert_array_equal(O.int_acc(xq, p, N), acc)
    ref = acc * (sa[:, None].astype(np.float64) / 127.0) * s[None, :]
    assert np.abs(of - ref).max() <= 4e-7 * np.abs(ref).max()
    np.testing.assert_array_equal(ob, O.f32_to_bf16(of))
    # VNNI u8 form == signed form whenever |sum (x+128) w| < 2^24
    u8 = (xq.astype(np.int64) + 128) @ q.astype(np.int64).T
    assert np.abs(u8).max() < 2 ** 24
    sb, sf = O.signed_linear(xq, sa, p, s, N)
    np.testing.assert_array_equal(sf, of)


@pytest.mark.parametrize("B", [64, 256])
def test_block_linear_closed_form(O, B):
    N, K, M = 32, 512, 3
    q, s = _quantized_linear(O, N, K, B)
    p, cs = O.pack_and_colsum(q, B, False)
    x = O.synth_normal_bf16(2, 1.0, (M, K))
    xq, sa = O.block_quant(x, B, True)
    ob, of = O.block_linear(xq, sa, p, s, cs, N, B)
    nb = K // B
    acc = np.einsum("mbk,nbk->mnb", xq.astype(np.int64).reshape(M, nb, B),
                    q.astype(np.int64).reshape(N, nb, B))
    ref = (acc * (sa[:, None, :].astype(np.float64) / 127.0)).sum(2) * s[None, :]
    assert np.abs(of - ref).max() <= 1e-6 * np.abs(ref).max()
    sb, sf = O.signed_block_linear(xq, sa, p, s, N, B)
    np.testing.assert_array_equal(sf, of)


def _f32(v):
    return np.float32(v)


def _bits(v):
    return int(np.array([v], np.float32).view(np.uint32)[0])


def test_exp_fast_coefficients(O):
    """exp_f32_fast (simd_math/ops.mojo:73-96) on |x| < ln2/2 has n = 0 and
    2^n = 1, so it is exactly its cubic 1 + r(c1 + r(c2 + r c3)) with r = x.
    Even and odd parts of oracle outputs at +-h recover the coefficients:
    p(h) + p(-h) = 2 + 2 c2 h^2 and (p(h) - p(-h)) / 2h = c1 + c3 h^2.  They
    must be the reference's 0.9999 / 0.4985 / 0.1681 (ops.mojo:88-90), not
    the Taylor 1 / 0.5 / 1/6 that the accurate exp_f32 approximates."""
    e = lambda v: float(O.lib().bqo_exp_f32_fast(float(v)))
    h1, h2 = 0.25, 0.125
    c2 = np.mean([(e(h) + e(-h) - 2.0) / (2 * h * h) for h in (h1, h2)])
    d1, d2 = ((e(h) - e(-h)) / (2 * h) for h in (h1, h2))
    c3 = (d1 - d2) / (h1 * h1 - h2 * h2)
    c1 = d2 - c3 * h2 * h2
    assert abs(c1 - 0.9999) < 2e-5, c1
    assert abs(c2 - 0.4985) < 2e-5, c2
    assert abs(c3 - 0.1681) < 2e-4, c3


def test_exp_fast_reduction_and_error(O):
    """Range reduction n = roundeven(x/ln2), r = x - n ln2, result p(r) 2^n
    (ops.mojo:83-95): fast(x) == fast(r) * 2^n exactly, with r the f32
    reduction; the input clamp at -87 (:82); and the error against exp is the
    polynomial's own, above the 1e-3 that an accurate exp would meet and
    below the documented ~0.3% (:76)."""
    lib = O.lib()
    LN2, INV_LN2 = _f32(0.6931471805599453), _f32(1.4426950408889634)
    for x in (-0.5, -1.0, -3.3, -7.0, -20.25, -60.0, -86.9):
        xf = _f32(x)
        n = int(np.rint(_f32(xf * INV_LN2)))
        r = _f32(xf - _f32(_f32(n) * LN2))
        assert abs(r) <= 0.35
        assert _f32(lib.bqo_exp_f32_fast(float(xf))) == _f32(lib.bqo_exp_f32_fast(float(r))) * _f32(2.0 ** n)
    assert lib.bqo_exp_f32_fast(-100.0) == lib.bqo_exp_f32_fast(-87.0)
    x = np.linspace(-87, 0, 20001).astype(np.float32)
    rel = np.abs(O.exp_fast(x).astype(np.float64) / np.exp(x.astype(np.float64)) - 1)
    assert 1e-3 < rel.max() < 4e-3, rel.max()


def test_tanh_gelu_closed_forms(O):
    """tanh_f32 (ops.mojo:128-141) is sign(x) (1 - E)/(1 + E) with E the
    pinned fast exp of -2|x|, and gelu_tanh_f32 (:145-156) is
    0.5 x (1 + tanh(0.7978845608 (x + 0.044715 x^3))) on that tanh, both in
    f32 with the reference's op order; exact tanh-GELU within 4e-3 |x|."""
    lib = O.lib()
    xs = np.concatenate([np.linspace(-12, 12, 4801), [0.0, -0.0, 1e-8, -3e-5, 40.0]]).astype(np.float32)
    for x in xs:
        E = _f32(lib.bqo_exp_f32_fast(float(_f32(-2.0) * _f32(abs(x)))))
        t = _f32(_f32(1.0 - E) / _f32(1.0 + E))
        t = -t if np.signbit(x) else t
        assert _bits(lib.bqo_tanh_f32(float(x))) == _bits(t), x
        x3 = _f32(_f32(x * x) * x)
        inner = _f32(_f32(0.7978845608028654) * _f32(x + _f32(_f32(0.044715) * x3)))
        g = _f32(_f32(_f32(0.5) * x) * _f32(1.0 + _f32(lib.bqo_tanh_f32(float(inner)))))
        assert _bits(lib.bqo_gelu_tanh_f32(float(x))) == _bits(g), x
    g = O.gelu_tanh(xs[:4801])
    xd = xs[:4801].astype(np.float64)
    exact = 0.5 * xd * (1 + np.tanh(math.sqrt(2 / math.pi) * (xd + 0.044715 * xd ** 3)))
    assert (np.abs(g - exact) <= 4e-3 * np.abs(xd) + 1e-6).all()


def test_gelu_gate_up_pins(O):
    """gelu_gate_up (elementwise.mojo:17-27) = bf16(gelu_tanh(gate) * up):
    with up = 1 it is bf16 of the pinned gelu_tanh of gate alone (a swapped
    gate/up would give gelu(1) * gate); gate = 10 gives exactly 10 * up
    (tanh rounds to 1); gate = 0 gives 0; and random operands stay within
    bf16 rounding of the exact tanh-GELU product."""
    rng = np.random.default_rng(3)
    g = O.f32_to_bf16(rng.normal(0, 2, 4096).astype(np.float32))
    one = np.full(4096, 0x3F80, np.uint16)
    np.testing.assert_array_equal(O.gelu_gate_up(g, one), O.f32_to_bf16(O.gelu_tanh(O.bf16_to_f32(g))))
    u = O.f32_to_bf16(rng.normal(0, 1, 4096).astype(np.float32))
    ten = np.full(4096, O.f32_to_bf16(np.float32([10.0]))[0], np.uint16)
    np.testing.assert_array_equal(O.gelu_gate_up(ten, u),
                                  O.f32_to_bf16(np.float32(10.0) * O.bf16_to_f32(u)))
    assert (O.bf16_to_f32(O.gelu_gate_up(np.zeros(4096, np.uint16), u)) == 0).all()
    gd, ud = O.bf16_to_f32(g).astype(np.float64), O.bf16_to_f32(u).astype(np.float64)
    exact = 0.5 * gd * (1 + np.tanh(math.sqrt(2 / math.pi) * (gd + 0.044715 * gd ** 3))) * ud
    got = O.bf16_to_f32(O.gelu_gate_up(g, u)).astype(np.float64)
    assert (np.abs(got - exact) <= 1e-2 * np.abs(exact) + 4e-3 * np.abs(gd * ud) + 1e-6).all()


def test_softmax_exp_known_values(O):
    """fast_exp_softmax_biased (simd_math/exponential.mojo:178-194) by hand:
    v = f32(12102203.16156148 x + 1059208216), i = trunc(v), k = the f32 with
    bits i, f = (i & 0x7FFFFF) / 2^23, result k (1.6501418 + f (-0.3755484 +
    f 0.3869647)).
      x =  0: v = 1059208192 = 0x3F223C00 (the bias rounded to f32's 64-step
              grid), k = 0.6337280, f = 0x223C00/2^23 = 0.2674561
              -> 0.99962980 (0x3F7FE7BD)
      x = -1: A x rounds to -12102203, v = 1047105989 -> f32 1047106048
              = 0x3E6991C0, k = 0.2280951, f = 0.8247604
              -> 0.36577994 (0x3EBB4782)
      x = -5: v = 998697177 -> f32 998697152 = 0x3B86E8C0, k = 0.0041171,
              f = 0.0539780 -> 0.0067149843 (0x3BDC095F)
    and within 1% of exp on the top-8 logit differences it sees (x > -60)."""
    lib = O.lib()
    for x, want in ((0.0, 0x3F7FE7BD), (-1.0, 0x3EBB4782), (-5.0, 0x3BDC095F)):
        assert _bits(lib.bqo_fast_exp_softmax_biased(x)) == want, (x, hex(_bits(lib.bqo_fast_exp_softmax_biased(x))))
    xs2 = np.linspace(-60, 0, 3001).astype(np.float32)
    sb = np.array([lib.bqo_fast_exp_softmax_biased(float(v)) for v in xs2])
    assert (np.abs(sb / np.exp(xs2.astype(np.float64)) - 1) < 1e-2).all()


def test_route_topk_softmax(O):
    logits = O.synth_normal_f32(2, 1.0, (64, 128))
    logits[0, 5] = logits[0, 9] = 10.0  # tie -> lower expert first
    idx, w = O.route_topk_softmax(logits, 8)
    ref = np.argsort(-logits, axis=1, kind="stable")[:, :8]
    np.testing.assert_array_equal(idx, ref)
    assert idx[0, 0] == 5 and idx[0, 1] == 9
    np.testing.assert_allclose(w.sum(1), 1.0, rtol=2e-6)
    assert (np.diff(w, axis=1) <= 1e-7).all()
    # the weights are a softmax over the k selected logits (not over all E):
    # fast_exp_softmax_biased is within 1% of exp, so within ~2% normalized
    top = np.take_along_axis(logits, idx, 1).astype(np.float64)
    sm = np.exp(top - top[:, :1])
    sm /= sm.sum(1, keepdims=True)
    assert (np.abs(w / sm - 1) < 2.5e-2).all()


def test_route_scale_and_sentinels(O):
    lib = O.lib()
    # out-of-range exponent inputs follow the x86 truncation (INT32_MIN -> -0.0)
    for v in (-1e30, -1e20, float("nan"), float("-inf")):
        r = lib.bqo_fast_exp_softmax_biased(v)
        assert r == 0.0 and math.copysign(1.0, r) < 0
    assert lib.bqo_fast_exp_softmax_biased(0.0) == pytest.approx(1.0, rel=1e-2)
    # per-expert scale multiplies the normalized weight once, in f32
    logits = O.synth_normal_f32(3, 1.0, (16, 32))
    scale = O.f32_to_bf16(1.0 + 0.5 * O.synth_normal_f32(4, 1.0, (32,)))
    idx, w = O.route_topk_softmax(logits, 4)
    idx_s, w_s = O.route_topk_softmax(logits, 4, per_expert_scale=scale)
    np.testing.assert_array_equal(idx_s, idx)
    np.testing.assert_array_equal(w_s, (w * O.bf16_to_f32(scale)[idx]).astype(np.float32))
    # fewer experts than k: the list is padded with {expert 0, -1e30}, whose
    # weight is -0.0
    idx3, w3 = O.route_topk_softmax(np.array([[0.5, 2.0, -1.0]], np.float32), 8)
    np.testing.assert_array_equal(idx3[0], [1, 0, 2, 0, 0, 0, 0, 0])
    assert (w3[0, 3:] == 0).all() and np.signbit(w3[0, 3:]).all()
    np.testing.assert_allclose(w3[0, :3].sum(), 1.0, rtol=1e-6)
    # logits at or below the sentinel, -inf and NaN never enter the list
    row = np.array([[np.nan, -np.inf, -1e30, -2e30, 1.0, np.nan, 3.0, -1e29]], np.float32)
    idx4, _ = O.route_topk_softmax(row, 4)
    np.testing.assert_array_equal(idx4[0], [6, 4, 7, 0])
    # no valid logit: k sentinels, each with fast_exp(0) / (k * fast_exp(0))
    idx5, w5 = O.route_topk_softmax(np.full((1, 6), np.nan, np.float32), 4)
    assert (idx5 == 0).all() and (w5 == w5[0, 0]).all()
    assert w5[0, 0] == pytest.approx(0.25, rel=1e-6)
    # -0.0 and +0.0 compare equal: the lower expert comes first
    idx6, _ = O.route_topk_softmax(np.array([[0.0, -1.0, -0.0, 0.0]], np.float32), 3)
    np.testing.assert_array_equal(idx6[0], [0, 2, 3])
    idx7, _ = O.route_topk_softmax(np.array([[-0.0, -1.0, 0.0]], np.float32), 2)
    np.testing.assert_array_equal(idx7[0], [0, 2])


def test_router_logits(O):
    rng = np.random.default_rng(6)
    T, H, E = 5, 256, 12
    x = O.f32_to_bf16(rng.standard_normal((T, H)).astype(np.float32))
    proj = O.f32_to_bf16(0.05 * rng.standard_normal((E, H)).astype(np.float32))
    rs = O.f32_to_bf16((1 + 0.2 * rng.standard_normal(H)).astype(np.float32))
    lg = O.router_logits(x, proj, rs)
    # float64 restatement of RMS-scale-and-project
    xd, pd, sd = (O.bf16_to_f32(a).astype(np.float64) for a in (x, proj, rs))
    sqrt_n, n_eps = O.norm_consts(H)
    inv = sqrt_n / np.sqrt((xd ** 2).sum(1) + n_eps)
    ref = (xd * sd * inv[:, None]) @ pd.T
    assert np.abs(lg - ref).max() <= 1e-5 * np.abs(ref).max()
    # one-hot projection rows pick single scaled elements exactly: pins the
    # element order of the chains (a transposed or shifted index picks another
    # element) and the scaling (x * scale) * inv_rms.  x in {+-1, +-2, +-0.5}
    # makes the sum of squares exact in any order.
    xs = O.f32_to_bf16(rng.choice([-2.0, -1.0, -0.5, 0.5, 1.0, 2.0], (T, H)).astype(np.float32))
    cols = np.array([0, 1, 15, 16, 17, 127, 128, 200, 255, 31, 64, 100])
    oh = np.zeros((E, H), np.float32)
    oh[np.arange(E), cols] = 1.0
    lg1 = O.router_logits(xs, O.f32_to_bf16(oh), rs)
    xf = O.bf16_to_f32(xs)
    ssq = (xf.astype(np.float64) ** 2).sum(1).astype(np.float32)
    inv32 = (np.float32(sqrt_n) / np.sqrt(ssq + np.float32(n_eps))).astype(np.float32)
    scaled = ((xf * O.bf16_to_f32(rs)[None, :]).astype(np.float32) * inv32[:, None]).astype(np.float32)
    np.testing.assert_array_equal(lg1, scaled[:, cols])


def test_build_schedule_vs_sort(O):
    rng = np.random.default_rng(4)
    T, k, E = 37, 4, 16
    idx = np.stack([rng.choice(E, k, replace=False) for _ in range(T)]).astype(np.int32)
    w = rng.random((T, k)).astype(np.float32)
    eo, routes = O.build_schedule(idx, w, E)
    order = sorted(((int(idx[t, j]), t, j) for t in range(T) for j in range(k)))
    np.testing.assert_array_equal(routes["token"], [t for _, t, _ in order])
    np.testing.assert_array_equal(routes["weight"], [w[t, j] for _, t, j in order])
    counts = np.bincount(idx.ravel(), minlength=E)
    np.testing.assert_array_equal(eo, np.concatenate([[0], np.cumsum(counts)]))


def _moe_case(O, T=6, E=4, k=2, H=128, I=64, seed=5):
    rng = np.random.default_rng(seed)
    idx = np.stack([rng.choice(E, k, replace=False) for _ in range(T)]).astype(np.int32)
    w = rng.random((T, k)).astype(np.float32)
    w /= w.sum(1, keepdims=True)
    eo, routes = O.build_schedule(idx, w, E)
    gu = O.bf16_to_f32(O.synth_normal_bf16(0, 0.02, (E * 2 * I, H)))
    gq, gs = O.rotate_and_quant(gu, 128 if H % 128 == 0 else 64)
    gp, gcs = O.pack_and_colsum(gq)
    dn = O.bf16_to_f32(O.synth_normal_bf16(9, 0.02, (E * H, I)))
    dq, ds = O.rotate_and_quant(dn, 64)
    dp, dcs = O.pack_and_colsum(dq, 64, False)
    x = O.synth_normal_bf16(1, 1.0, (T, H))
    xq, xsa = O.norm_quant(x, np.full(H, 0x3F80, np.uint16), 64)
    return dict(idx=idx, w=w, eo=eo, routes=routes, gq=gq, gs=gs, gp=gp, gcs=gcs, dq=dq, ds=ds,
                dp=dp, dcs=dcs, xq=xq, xsa=xsa, T=T, E=E, k=k, H=H, I=I)


def test_moe_phases_closed_form(O):
    c = _moe_case(O)
    T, E, H, I = c["T"], c["E"], c["H"], c["I"]
    bucket = O.moe_phase1(c["xq"], c["xsa"], c["eo"], c["routes"], c["gp"], c["gs"], c["gcs"], I)
    gq = c["gq"].astype(np.int64).reshape(E, 2 * I, H)
    ref = np.zeros((len(c["routes"]), I))
    for e in range(E):
        for rec in range(c["eo"][e], c["eo"][e + 1]):
            t = c["routes"]["token"][rec]
            a = gq[e] @ c["xq"][t].astype(np.int64)
            v = a * (c["xsa"][t] / 127.0) * c["gs"][e * 2 * I:(e + 1) * 2 * I]
            g, u = v[:I], v[I:]
            ref[rec] = 0.5 * g * (1 + np.tanh(math.sqrt(2 / math.pi) * (g + 0.044715 * g ** 3))) * u
    got = O.bf16_to_f32(bucket).astype(np.float64)
    assert np.abs(got - ref).max() <= 1e-2 * np.abs(ref).max()
    bq_, bsa = O.block_quant(bucket, 64, True)
    accum, out = O.moe_phase2(bq_, bsa, c["eo"], c["routes"], T, c["dp"], c["ds"], c["dcs"], H)
    dq = c["dq"].astype(np.int64).reshape(E, H, I)
    ref2 = np.zeros((T, H))
    for e in range(E):
        for rec in range(c["eo"][e], c["eo"][e + 1]):
            t = c["routes"]["token"][rec]
            acc = np.einsum("nbk,bk->nb", dq[e].reshape(H, I // 64, 64),
                            bq_[rec].astype(np.int64).reshape(I // 64, 64))
            y = (acc * (bsa[rec] / 127.0)).sum(1) * c["ds"][e * H:(e + 1) * H]
            ref2[t] += y * c["routes"]["weight"][rec]
    assert np.abs(accum - ref2).max() <= 1e-5 * np.abs(ref2).max()
    np.testing.assert_array_equal(out, O.f32_to_bf16(accum))


def test_synth_normal(O):
    x = O.synth_normal_f32(0, 0.02, (200000,))
    assert abs(x.mean()) < 2e-4 and abs(x.std() - 0.02) < 2e-4
    b = O.synth_normal_bf16(0, 0.02, (1001,))
    np.testing.assert_array_equal(b, O.f32_to_bf16(O.synth_normal_f32(0, 0.02, (1001,))))


# ---------------------------------------------------------------- head / embedding
def test_sampling_rng_and_math(O):
    L = O.lib()
    # SplitMix64 from state 0 publishes 0xE220A8397B1DCDAF, 0x6E789E6AA1B965F4,
    # 0x06C45D188009454F: the finalizer of gamma, 2*gamma, 3*gamma
    gamma = 0x9E3779B97F4A7C15
    assert L.bqo_mix64(0) == 0xE220A8397B1DCDAF
    assert L.bqo_mix64(gamma) == 0x6E789E6AA1B965F4
    assert L.bqo_mix64((2 * gamma) % (1 << 64)) == 0x06C45D188009454F
    # exp_f32 / log_f32 against libm; the exp clamp at -87 / 88
    xs = np.linspace(-87, 88, 2001).astype(np.float32)
    e = np.array([L.bqo_exp_f32(float(v)) for v in xs])
    assert (np.abs(e / np.exp(xs.astype(np.float64)) - 1) < 2e-6).all()
    assert L.bqo_exp_f32(-100.0) == L.bqo_exp_f32(-87.0)
    ls = np.exp(np.linspace(-60, 60, 2001)).astype(np.float32)
    lg = np.array([L.bqo_log_f32(float(v)) for v in ls])
    assert (np.abs(lg - np.log(ls.astype(np.float64))) < 2e-6 * np.maximum(1, np.abs(lg))).all()
    # Gumbel(0, 1): mean = Euler-Mascheroni, variance = pi^2/6, CDF exp(-exp(-x))
    g = np.array([L.bqo_gumbel_noise(11, 3, i) for i in range(200000)])
    assert abs(g.mean() - 0.5772156649) < 0.01 and abs(g.var() - math.pi ** 2 / 6) < 0.03
    for q in (-1.0, 0.0, 1.0, 3.0):
        assert abs((g <= q).mean() - math.exp(-math.exp(-q))) < 0.005
    # different rows / seeds give different streams
    assert L.bqo_gumbel_noise(11, 4, 5) != L.bqo_gumbel_noise(11, 3, 5)
    assert L.bqo_gumbel_noise(12, 3, 5) != L.bqo_gumbel_noise(11, 3, 5)
    # softcap: tanh(x/c)*c with the fast tanh
    for v in (-100.0, -3.0, 0.5, 29.0, 1000.0):
        assert abs(L.bqo_softcap(v, 30.0) - 30 * math.tanh(v / 30)) < 3e-3 * 30


def _head_case(O, R, V, H, seed, block=128, spread=1.0):
    rng = np.random.default_rng(seed)
    x = O.f32_to_bf16(rng.standard_normal((R, H)).astype(np.float32))
    xq, xsa = O.norm_quant(x, np.full(H, 0x3F80, np.uint16), block, per_block=True)
    w = rng.integers(-127, 128, (V, H), dtype=np.int8)
    ws = (spread * rng.random((V, H // block)) / 127 / 40).astype(np.float32)
    return xq, xsa, w, ws


def test_head_logit_row(O):
    rng = np.random.default_rng(3)
    H, B = 512, 128
    x = rng.integers(-127, 128, H, dtype=np.int8)
    w = rng.integers(-127, 128, H, dtype=np.int8)
    # sa = 127, scale = 1: the f32 chain sums exact integers (< 2^24)
    f = O.lib().bqo_head_logit_row
    f.restype = C.c_float
    f.argtypes = [C.c_void_p] * 4 + [C.c_int, C.c_int]
    ones = np.ones(H // B, np.float32)
    got = f(x.ctypes.data, (127 * ones).ctypes.data, w.ctypes.data, ones.ctypes.data, H, B)
    assert got == float(np.dot(x.astype(np.int64), w.astype(np.int64)))
    sa = rng.random(H // B).astype(np.float32) * 4
    ws = rng.random(H // B).astype(np.float32) * 0.01
    got = f(x.ctypes.data, sa.ctypes.data, w.ctypes.data, ws.ctypes.data, H, B)
    blocks = (x.astype(np.int64) * w).reshape(-1, B).sum(1)
    ref = float((blocks * (sa.astype(np.float64) / 127) * ws).sum())
    assert abs(got - ref) <= 1e-5 * abs(ref)


def test_flash_sample_greedy_and_filters(O):
    R, V, H = 3, 2048, 256
    xq, xsa, w, ws = _head_case(O, R, V, H, 5)
    p = O.sampling_params(R, temperature=[1.0, 0.5, 2.0], greedy=True)
    out = O.flash_sample(xq, xsa, w, ws, p)
    # y for every (row, v) from the per-row function + softcap + bf16
    L = O.lib()
    f = L.bqo_head_logit_row
    f.restype = C.c_float
    f.argtypes = [C.c_void_p] * 4 + [C.c_int, C.c_int]
    y = np.zeros((R, V), np.float32)
    for r in range(R):
        for v in range(V):
            raw = f(xq[r].ctypes.data, xsa[r].ctypes.data, w[v].ctypes.data, ws[v].ctypes.data, H, 128)
            y[r, v] = O.bf16_to_f32(O.f32_to_bf16(np.array([L.bqo_softcap(raw, 30.0)], np.float32)))[0]
    for r in range(R):
        order = np.lexsort((np.arange(V), -y[r]))   # y descending, lower index first
        assert out["n"][r] == 256
        np.testing.assert_array_equal(out["topn_idx"][r], order[:256])
        np.testing.assert_array_equal(out["topn_val"][r], y[r, order[:256]])
        assert out["token_id"][r] == order[0]       # greedy: the first maximum
        T = p["temperature"][r]
        yt = y[r].astype(np.float64) * np.float64(np.float32(1) / np.float32(T))
        lse = yt.max() + np.log(np.exp(yt - yt.max()).sum())
        assert abs(out["logz"][r] - lse) < 1e-5 * abs(lse) + 1e-5
    # top_k = 1 picks the top logit; n_keep truncates; min_p = 1 keeps only
    # the maximal value
    p2 = O.sampling_params(R, seed=[7, 8, 9], top_k=[1, 0, 0], n_keep=[256, 10, 256],
                           min_p=[0.0, 0.0, 1.0])
    out2 = O.flash_sample(xq, xsa, w, ws, p2)
    assert out2["token_id"][0] == out["topn_idx"][0][0]
    assert out2["n"][1] == 10 and (out2["topn_idx"][1][10:] == -1).all()
    assert (out2["topn_val"][1][10:] == np.float32(-1e30)).all()
    top2 = out2["topn_idx"][2]
    assert y[2, out2["token_id"][2]] == y[2, top2[0]]
    # without filters the token is the argmax of y/T + gumbel (first on ties)
    for r in (1,):
        g = np.array([L.bqo_gumbel_noise(int(p2["seed"][r]), r, v) for v in range(V)], np.float32)
        score = (y[r] * (np.float32(1) / np.float32(p2["temperature"][r]))).astype(np.float32) + g
        assert out2["token_id"][r] == int(np.argmax(score))


def test_embed_lookup(O):
    rng = np.random.default_rng(8)
    rows, H, B = 64, 512, 128
    w = np.zeros((rows, H), np.int8)
    ws = (rng.random((rows, H // B)) + 0.5).astype(np.float32)
    w[3, 130] = 5            # a single code in block 1 of row 3
    w[7] = rng.integers(-127, 128, H, dtype=np.int8)
    tok = np.array([3, 7, 70, 3], np.int32)  # 70 belongs to shard 1
    scale = O.embed_scale(2816)
    assert scale == 53.0
    out = O.bf16_to_f32(O.embed_lookup(tok, w, ws, B, scale=scale))
    # FWHT of a one-hot: +-c_B everywhere in that block, zero elsewhere
    c = O.fwht_scale(B)
    k = np.arange(B)
    sign = np.where([bin(v & (130 - B)).count("1") % 2 for v in k], -1.0, 1.0)
    ref = np.float32(5 * ws[3, 1]) * np.float32(c) * sign
    ref = O.bf16_to_f32(O.f32_to_bf16((ref.astype(np.float32) * np.float32(scale)).astype(np.float32)))
    np.testing.assert_array_equal(out[0, B:2 * B], ref)
    assert (out[0, :B] == 0).all() and (out[0, 2 * B:] == 0).all()
    assert (out[2] == 0).all()                 # foreign shard: zero row
    np.testing.assert_array_equal(out[3], out[0])
    # a generic row against the float64 rotation
    deq = w[7].astype(np.float64).reshape(-1, B) * ws[7][:, None]
    hd = np.array([[(-1) ** bin(i & j).count("1") for j in range(B)] for i in range(B)], np.float64)
    rot = (deq @ hd.T / math.sqrt(B)).reshape(-1) * scale
    assert np.abs(out[1] - rot).max() <= 2 ** -7 * np.abs(rot).max()
    # sharded: rank 1 of two owns rows [32, 64)
    out_r1 = O.embed_lookup(np.array([40, 3], np.int32), w[32:], ws[32:], B, scale=scale,
                            shard_rows=32, rank=1)
    assert (out_r1[1] == 0).all()
    np.testing.assert_array_equal(out_r1[0], O.embed_lookup(np.array([40], np.int32), w, ws, B,
                                                            scale=scale)[0])
    # the owner is Mojo's floor division (embedding.mojo:42): negative ids
    # (padding) belong to no rank >= 0, ids past the last shard to none either
    odd = np.array([-1, -32, -33, -(2 ** 31), 64, 10 ** 6, 7], np.int32)
    for rank in (0, 1):
        o = O.embed_lookup(odd, w[32 * rank:32 * rank + 32], ws[32 * rank:32 * rank + 32], B,
                           scale=scale, shard_rows=32, rank=rank)
        assert (o[:6] == 0).all()
        assert (o[6] != 0).any() == (rank == 0)


def test_head_prep_per_block(O):
    # per-block head prep: block == hidden reproduces the per-row norm-quant;
    # every block's amax maps to +-127
    rng = np.random.default_rng(9)
    H = 512
    x = O.f32_to_bf16(rng.standard_normal((4, H)).astype(np.float32))
    g = np.full(H, 0x3F80, np.uint16)
    q1, s1 = O.norm_quant(x, g, 512)
    q2, s2 = O.norm_quant(x, g, 512, per_block=True)
    np.testing.assert_array_equal(q1, q2)
    np.testing.assert_array_equal(s1, s2[:, 0])
    q3, s3 = O.norm_quant(x, g, 128, per_block=True)
    assert s3.shape == (4, 4)
    assert (np.abs(q3.reshape(4, 4, 128)).max(2) == 127).all()
