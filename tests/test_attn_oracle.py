"""Pins of the oracle's int8-KV attention (oracle/bq_oracle.c bqo_attn_prep,
bqo_flash_attention; reference butterquant/head_prep.mojo:9-92,
butterquant_kernels/attention.mojo:32-534, kernels/attention_ops.mojo:45-182,
kernels/logsum_merge.mojo:29-122).  The reference holds no golden vectors
for this path; its own attention tests (tests/test_*_attention_degree_parity
.mojo) are self-consistency checks across degrees.  So the oracle is pinned
by:
  - the prep against a float64 pipeline (RMS, gain, RoPE as a rotation,
    FWHT as the normalized Hadamard matrix, round-to-nearest codes);
  - where the prep writes: the page-table closed form, cache_degree/rank;
  - the attention's f32 values against a float64 closed form of the
    online-softmax recursion (every tile's weights times the product of the
    later tiles' corrections, the splits combined with their corrections),
    and against plain float64 softmax attention (the reference's fast exp
    is ~0.5% off exp, so that comparison is loose);
  - exact invariances: page permutation, positions outside the window or in
    the future, doubling every V scale, swapping KV heads.
"""
import ctypes as C

import numpy as np
import pytest

from attn_cases import make_case, oracle_attention, run_index


def hadamard(n):
    h = np.array([[1.0]])
    while h.shape[0] < n:
        h = np.block([[h, h], [h, -h]])
    return h / np.sqrt(n)


def rope_tables(maxpos, rope_half, theta=10000.0):
    inv = 1.0 / theta ** (np.arange(rope_half) / rope_half)
    ang = np.arange(maxpos)[:, None] * inv[None, :]
    return np.cos(ang).astype(np.float32), np.sin(ang).astype(np.float32)


def prep_f64(x, gamma, cs, sn, hd, rope_half, ps, sqrt_n, n_eps):
    x = x.astype(np.float64)
    inv = float(sqrt_n) / np.sqrt((x * x).sum() + float(n_eps))
    y = x * inv
    if gamma is not None:
        y = y * gamma
        lo, hi = y[:rope_half].copy(), y[ps:ps + rope_half].copy()
        y[:rope_half] = lo * cs - hi * sn
        y[ps:ps + rope_half] = hi * cs + lo * sn
    y = hadamard(hd) @ y
    amax = max(np.abs(y).max(), 1e-10)
    return y * (127.0 / amax), amax


@pytest.mark.parametrize("hd,rope_half,ps", [(256, 128, 128), (512, 64, 256), (128, 64, 64)])
def test_prep_against_f64(O, hd, rope_half, ps):
    rng = np.random.default_rng(hd + rope_half)
    nq, nkv, T = 4, 2, 3
    q = O.f32_to_bf16(rng.standard_normal((T, nq * hd)).astype(np.float32) * 3)
    k = O.f32_to_bf16(rng.standard_normal((T, nkv * hd)).astype(np.float32))
    v = O.f32_to_bf16(rng.standard_normal((T, nkv * hd)).astype(np.float32) * 0.2)
    qn = O.f32_to_bf16(rng.uniform(0.5, 1.5, hd).astype(np.float32))
    kn = O.f32_to_bf16(rng.uniform(0.5, 1.5, hd).astype(np.float32))
    cos, sin = rope_tables(64, rope_half)
    page = 16
    kc = np.zeros((4 * page, nkv * hd), np.int8); vc = np.zeros_like(kc)
    ks = np.zeros((4 * page, nkv), np.float32); vs = np.zeros_like(ks)
    runs = O.kv_runs([(0, 37, 0, 3)])
    rows = np.array([2 * page, 0, 3 * page], np.int32)
    qi, qb, fq = O.attn_prep(q, k, v, qn, kn, kc, ks, vc, vs, cos, sin, runs, rows, nq, nkv, hd,
                             rope_half, ps, 4, page - 1, -1)
    sqrt_n, n_eps = O.norm_consts(hd)
    g_q, g_k = O.bf16_to_f32(qn).astype(np.float64), O.bf16_to_f32(kn).astype(np.float64)
    checked = mism = 0

    def check(codes, scale, x, gamma, pos):
        nonlocal checked, mism
        y, amax = prep_f64(O.bf16_to_f32(x), gamma, cos[pos], sin[pos], hd, rope_half, ps,
                           sqrt_n, n_eps)
        assert scale == pytest.approx(amax, rel=1e-5)
        ref = np.clip(np.round(y), -128, 127)
        d = np.abs(codes.astype(np.float64) - ref)
        frac = np.abs(y - np.floor(y) - 0.5)
        assert (d <= 1).all()
        assert (frac[d > 0] < 2e-3).all(), "a code differs away from a rounding tie"
        checked += hd
        mism += int((d > 0).sum())

    for t in range(T):
        pos = 37 + t
        for h in range(nq):
            codes = qi[t, h * hd:(h + 1) * hd]
            check(codes, fq[t, h], q[t, h * hd:(h + 1) * hd], g_q, pos)
            assert qb[t, h] == 128.0 * codes.astype(np.int64).sum()
        slot = int(rows[(pos >> 4)]) + (pos & 15)
        for h in range(nkv):
            check(kc[slot, h * hd:(h + 1) * hd], ks[slot, h], k[t, h * hd:(h + 1) * hd], g_k, pos)
            check(vc[slot, h * hd:(h + 1) * hd], vs[slot, h], v[t, h * hd:(h + 1) * hd], None, pos)
    assert mism <= checked // 500


def test_prep_cache_rows_and_rank(O):
    # two runs, shuffled pages, K/V for positions of cache rank 1 of 2 only
    rng = np.random.default_rng(5)
    hd, nq, nkv, page = 64, 2, 1, 8
    seqs = [(5, 6), (30, 4)]
    T = sum(n for _, n in seqs)
    x = lambda n: O.f32_to_bf16(rng.standard_normal((T, n)).astype(np.float32))
    q, k, v = x(nq * hd), x(nkv * hd), x(nkv * hd)
    one = np.full(hd, 0x3F80, np.uint16)
    cos, sin = rope_tables(64, 0)
    slots = 10 * page
    kc = np.zeros((slots, hd), np.int8); vc = np.zeros_like(kc)
    ks = np.zeros((slots, 1), np.float32); vs = np.zeros_like(ks)
    runs = O.kv_runs([(0, 5, 0, 2), (6, 30, 2, 3)])
    rows = np.array([7 * page, 2 * page, 0, 9 * page, 4 * page], np.int32)
    O.attn_prep(q, k, v, one, one, kc, ks, vc, vs, cos, sin, runs, rows, nq, nkv, hd, 0, 0, 3,
                page - 1, -1, cache_degree=2, rank=1)
    expect = set()
    for r, (base, n) in enumerate(seqs):
        for t in range(n):
            pos = base + t
            if pos % 2 == 1:
                p = pos // 2
                expect.add(int(rows[runs[r]["rows_off"] + (p >> 3)]) + (p & 7))
    written = set(np.nonzero(ks[:, 0])[0].tolist())
    assert written == expect
    assert set(np.nonzero(vs[:, 0])[0].tolist()) == expect
    untouched = np.setdiff1d(np.arange(slots), list(expect))
    assert not kc[untouched].any() and not vc[untouched].any()


_fexp = None


def fexp(x):
    global _fexp
    if _fexp is None:
        import oracle
        _fexp = oracle.lib().bqo_fast_exp_softmax_biased
        _fexp.restype, _fexp.argtypes = C.c_float, [C.c_float]
    return np.array([_fexp(float(v)) for v in np.ravel(x)], np.float64).reshape(np.shape(x))


def scores_f32(c, tok, h, ps_):
    """f32 scores of query head h against positions ps_ (the reference's
    op order: ((dot * f_q) * ks) / 127^2)."""
    hd, g = c.head_dim, c.num_q // c.num_kv
    q = c.q_i8[tok, h * hd:(h + 1) * hd].astype(np.int64)
    inv = np.float32(1.0) / np.float32(127.0)
    out = []
    for p in ps_:
        s = c.slot(tok, p)
        kh = c.k_cache[s, (h // g) * hd:(h // g + 1) * hd].astype(np.int64)
        v = np.float32((kh * q).sum()) * c.f_q[tok, h]
        out.append(np.float32(np.float32(v * c.k_scale[s, h // g]) * np.float32(inv * inv)))
    return np.array(out, np.float32)


def closed_form(O, c, tok, h, s_max):
    """float64 closed form of the online recursion and the merge."""
    hd, g = c.head_dim, c.num_q // c.num_kv
    lo, hi = c.kv_range(tok)
    L = hi - lo
    S = O.attn_num_splits(L, s_max, 32)
    per = (L + S - 1) // S
    parts = []
    for s in range(S):
        a, e = min(s * per, L), min(s * per + per, L)
        M = np.float32(-1e30)
        tiles = []
        for p0 in range(a, e, 16):
            tl = min(16, e - p0)
            sc = np.full(16, np.float32(-1e30), np.float32)
            sc[:tl] = scores_f32(c, tok, h, range(lo + p0, lo + p0 + tl))
            Mn = max(M, sc.max())
            corr = fexp(max(np.float32(M - Mn), np.float32(-87)))
            w = fexp(np.maximum(sc - Mn, np.float32(-87)))
            tiles.append((p0, tl, corr, w))
            M = Mn
        acc = np.zeros(hd)
        lsum = 0.0
        for u, (p0, tl, _, w) in enumerate(tiles):
            later = np.prod([t[2] for t in tiles[u + 1:]]) if u + 1 < len(tiles) else 1.0
            W = w * later
            lsum += W.sum()
            for t in range(tl):
                sl = c.slot(tok, lo + p0 + t)
                vv = c.v_cache[sl, (h // g) * hd:(h // g + 1) * hd].astype(np.float64)
                acc += W[t] * vv * float(c.v_scale[sl, h // g]) / 127.0
        parts.append((M, lsum, acc))
    if c.window > 0 and S == 1:
        m, lsum, acc = parts[0]
        return acc / lsum
    gm = max(p[0] for p in parts)
    num, den = np.zeros(hd), 0.0
    for m, lsum, acc in parts:
        if lsum > 0:
            cs = fexp(max(np.float32(m - gm), np.float32(-87)))
            num += cs * acc
            den += cs * lsum
    return num / den


def softmax_f64(c, tok, h):
    hd, g = c.head_dim, c.num_q // c.num_kv
    lo, hi = c.kv_range(tok)
    q = c.q_i8[tok, h * hd:(h + 1) * hd].astype(np.float64)
    sc, vals = [], []
    for p in range(lo, hi):
        s = c.slot(tok, p)
        kh = c.k_cache[s, (h // g) * hd:(h // g + 1) * hd].astype(np.float64)
        sc.append((kh @ q) * c.f_q[tok, h] * c.k_scale[s, h // g] / 127.0 ** 2)
        vals.append(c.v_cache[s, (h // g) * hd:(h // g + 1) * hd] * (c.v_scale[s, h // g] / 127.0))
    sc = np.array(sc)
    w = np.exp(sc - sc.max())
    return (w[:, None] * np.array(vals)).sum(0) / w.sum()


CASES = {
    # sliding decode batch: one token per run, short and full windows (ring pages wrap)
    "sliding_decode": dict(num_q=4, num_kv=2, head_dim=128, page_len=64, window=100,
                           seqs=[(3, 1), (70, 1), (230, 1)]),
    # sliding prefill chunk continuing a sequence
    "sliding_prefill": dict(num_q=2, num_kv=1, head_dim=64, page_len=32, window=40,
                            seqs=[(50, 9)]),
    # full attention, two sequences, GQA 4
    "full": dict(num_q=8, num_kv=2, head_dim=64, page_len=16, seqs=[(0, 3), (90, 2)]),
}


@pytest.mark.parametrize("name", sorted(CASES))
@pytest.mark.parametrize("s_max", [1, 4])
def test_attention_closed_form(O, name, s_max):
    c = make_case(O, 11, **CASES[name])
    out, o32 = oracle_attention(O, c, s_max=s_max, with_f32=True)
    hd = c.head_dim
    for tok in range(c.T):
        for h in range(c.num_q):
            ref = closed_form(O, c, tok, h, s_max)
            got = o32[tok, h * hd:(h + 1) * hd].astype(np.float64)
            assert np.abs(got - ref).max() <= 2e-5 * np.abs(ref).max(), (tok, h)
            # within the reference's fast exp of exact softmax attention
            soft = softmax_f64(c, tok, h)
            assert np.abs(got - soft).max() <= 3e-2 * np.abs(soft).max(), (tok, h)
    np.testing.assert_array_equal(out, O.f32_to_bf16(o32))


def test_attention_invariances(O):
    base = dict(num_q=4, num_kv=2, head_dim=64, page_len=16, window=30, seqs=[(40, 4), (7, 1)])
    c = make_case(O, 3, **base)
    ref = oracle_attention(O, c, s_max=2)
    hd = c.head_dim

    # 1. page permutation: move every page, rewrite base_rows
    npg = c.k_cache.shape[0] // 16
    perm = np.random.default_rng(9).permutation(npg)
    c2 = make_case(O, 3, **base)
    for name in ("k_cache", "v_cache", "k_scale", "v_scale"):
        a = getattr(c, name)
        b = np.empty_like(a)
        for old in range(npg):
            b[perm[old] * 16:(perm[old] + 1) * 16] = a[old * 16:(old + 1) * 16]
        setattr(c2, name, b)
    c2.base_rows = (perm[c.base_rows // 16] * 16).astype(np.int32)
    np.testing.assert_array_equal(oracle_attention(O, c2, s_max=2), ref)

    # 2. rows no token reads (outside every window, or later positions) do not matter
    used = {c.slot(t, p) for t in range(c.T) for p in range(*c.kv_range(t))}
    free = np.setdiff1d(np.arange(c.k_cache.shape[0]), sorted(used))
    assert len(free) > 0
    c3 = make_case(O, 3, **base)
    c3.k_cache[free] = -c3.k_cache[free]
    c3.v_cache[free] = 7
    c3.k_scale[free] *= 3
    np.testing.assert_array_equal(oracle_attention(O, c3, s_max=2), ref)
    # ... while the first row inside token 0's window does
    lo, _ = c.kv_range(0)
    c4 = make_case(O, 3, **base)
    c4.v_cache[c.slot(0, lo)] = -c4.v_cache[c.slot(0, lo)]
    assert (oracle_attention(O, c4, s_max=2)[0] != ref[0]).any()

    # 3. doubling every V scale doubles every output exactly
    c5 = make_case(O, 3, **base)
    c5.v_scale *= 2
    np.testing.assert_array_equal(O.bf16_to_f32(oracle_attention(O, c5, s_max=2)),
                                  2 * O.bf16_to_f32(ref))

    # 4. q head h reads kv head h // (num_q/num_kv): swap the kv heads' data
    c6 = make_case(O, 3, **base)
    for name in ("k_cache", "v_cache"):
        a = getattr(c6, name)
        a[:, :hd], a[:, hd:] = a[:, hd:].copy(), a[:, :hd].copy()
    for name in ("k_scale", "v_scale"):
        a = getattr(c6, name)
        a[:, [0, 1]] = a[:, [1, 0]]
    g = c.num_q // c.num_kv
    qs = c6.q_i8.reshape(c.T, c.num_q, hd)
    c6.q_i8 = np.ascontiguousarray(np.concatenate([qs[:, g:], qs[:, :g]], 1).reshape(c.T, -1))
    c6.f_q = np.ascontiguousarray(np.concatenate([c6.f_q[:, g:], c6.f_q[:, :g]], 1))
    c6.qi_bias = np.ascontiguousarray(np.concatenate([c6.qi_bias[:, g:], c6.qi_bias[:, :g]], 1))
    got = oracle_attention(O, c6, s_max=2).reshape(c.T, c.num_q, hd)
    r = ref.reshape(c.T, c.num_q, hd)
    np.testing.assert_array_equal(got[:, g:], r[:, :g])
    np.testing.assert_array_equal(got[:, :g], r[:, g:])


def test_split_plan(O):
    # worker_range parts of ceil(L/32) or s_max pieces
    assert O.attn_num_splits(1, 8, 32) == 1
    assert O.attn_num_splits(33, 8, 32) == 2
    assert O.attn_num_splits(1024, 8, 32) == 8
    assert O.attn_num_splits(0, 8, 32) == 1
    c = make_case(O, 1, num_q=2, num_kv=1, head_dim=64, page_len=16, seqs=[(0, 1)])
    assert run_index(c.runs, 0) == 0
