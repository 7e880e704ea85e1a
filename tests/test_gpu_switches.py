"""GPU parity of the library's non-default tuning paths (BQ_* switches read at
bq_init), each against the CPU oracle, bit-exact: every switch value the
library still accepts selects a code path that stays correct.  The default
paths are covered by the other GPU tests."""
import numpy as np
import pytest

from test_gpu_parity import _dense_gate_up_ref, dev, host, weight

pytestmark = pytest.mark.gpu
ONE = 0x3F80


# ------------------------------------------------------- decode GEMV waves
@pytest.mark.parametrize("waves", [4, 8, 16])
@pytest.mark.parametrize("M,K", [(1, 4096), (1, 2816), (3, 2816), (16, 4096), (16, 8192),
                                 (5, 1024)])
def test_gemv_waves_per_row(gpu, O, tune_env, waves, M, K):
    tune_env(BQ_GEMV_WAVES=waves)
    N = 128
    q, s, W = weight(gpu, O, N, K, 128)
    p, cs = O.pack_and_colsum(q)
    x = O.synth_normal_bf16(1, 1.0, (M, K))
    xq, sa = O.norm_quant(x, np.full(K, ONE, np.uint16), 128)
    ob, of = gpu.linear(dev(xq), dev(sa), W, want_f32=True)
    rb, rf = O.linear(xq, sa, p, s, cs, N)
    np.testing.assert_array_equal(host(of), rf)
    np.testing.assert_array_equal(host(ob), rb)


@pytest.mark.parametrize("waves", [0, 2, 4, 8])
@pytest.mark.parametrize("K", [64, 128, 192, 1024, 2816, 4096, 8192])
def test_gemv_m1_waves(gpu, O, tune_env, waves, K):
    """M = 1 per-row (k_gemv_m1 up to K = 4096, the general kernel above; 0 =
    the default wave count): small K leaves some waves no k-step."""
    tune_env(BQ_GEMV_M1_WAVES=waves)
    N, B = 96, min(K, 128) if K % 128 == 0 else 64
    q, s, W = weight(gpu, O, N, K, B, seed=8)
    p, cs = O.pack_and_colsum(q)
    x = O.synth_normal_bf16(9, 1.0, (1, K))
    xq, sa = O.norm_quant(x, np.full(K, ONE, np.uint16), B)
    ob, of = gpu.linear(dev(xq), dev(sa), W, want_f32=True)
    rb, rf = O.linear(xq, sa, p, s, cs, N)
    np.testing.assert_array_equal(host(of), rf)
    np.testing.assert_array_equal(host(ob), rb)


@pytest.mark.parametrize("waves", [2, 4, 8])
def test_gemv_m1_segments(gpu, O, tune_env, waves):
    """q/k/v of one token in one k_gemv_m1 launch: each segment = the oracle."""
    tune_env(BQ_GEMV_M1_WAVES=waves)
    K = 2816
    ws = [weight(gpu, O, n, K, 128, seed=sd) for n, sd in ((256, 1), (128, 2), (128, 3))]
    x = O.synth_normal_bf16(10, 1.0, (1, K))
    xq, sa = O.norm_quant(x, np.full(K, ONE, np.uint16), 128)
    outs = gpu.qkv(dev(xq), dev(sa), *(w[2] for w in ws))
    for o, (q, s, _) in zip(outs, ws):
        p, cs = O.pack_and_colsum(q)
        rb, _ = O.linear(xq, sa, p, s, cs, q.shape[0])
        np.testing.assert_array_equal(host(o), rb)


@pytest.mark.parametrize("waves", [4, 8, 16])
@pytest.mark.parametrize("M,K,B", [(1, 2112, 64), (16, 2112, 64), (16, 4096, 256),
                                   (7, 8192, 512), (16, 4096, 512), (2, 2816, 256)])
def test_gemv_waves_per_block(gpu, O, tune_env, waves, M, K, B):
    tune_env(BQ_GEMV_WAVES=waves)
    N = 128
    q, s, W = weight(gpu, O, N, K, B, seed=4)
    p, cs = O.pack_and_colsum(q, B, False)
    x = O.synth_normal_bf16(5, 1.0, (M, K))
    xq, sa = O.block_quant(x, B, B == 64)
    ob, of = gpu.block_linear(dev(xq), dev(sa), W, B, want_f32=True)
    rb, rf = O.block_linear(xq, sa, p, s, cs, N, B)
    np.testing.assert_array_equal(host(of), rf)
    np.testing.assert_array_equal(host(ob), rb)



# ------------------------------------------------------------ norm-quant forms
@pytest.mark.parametrize("sw", [dict(BQ_NQ_PAIR=0), dict(BQ_NQ_V8=0),
                                dict(BQ_NQ_PAIR=0, BQ_NQ_V8=0)])
@pytest.mark.parametrize("T,H,B", [(1, 2816, 128), (5, 4096, 128), (259, 2816, 128),
                                   (1795, 2816, 128), (3, 3072, 256), (300, 2048, 512)])
def test_norm_quant_switches(gpu, O, tune_env, sw, T, H, B):
    tune_env(**sw)
    x = O.synth_normal_bf16(11, 1.0, (T, H))
    g = O.f32_to_bf16(O.synth_normal_f32(12, 0.3, (H,)) + 1.0)
    q, sa = gpu.norm_quant(dev(x), dev(g), B)
    rq, rsa = O.norm_quant(x, g, B)
    np.testing.assert_array_equal(host(sa), rsa)
    np.testing.assert_array_equal(host(q), rq)


@pytest.mark.parametrize("sw", [dict(BQ_NQ_PAIR=0), dict(BQ_NQ_V8=0)])
@pytest.mark.parametrize("K,B", [(2816, 128), (4096, 256)])
def test_norm_linear_switches(gpu, O, tune_env, sw, K, B):
    tune_env(**sw)
    N = 256
    q, s, W = weight(gpu, O, N, K, 128, seed=3)
    p, cs = O.pack_and_colsum(q)
    x = O.synth_normal_bf16(7, 1.0, (1, K))
    g = O.f32_to_bf16(O.synth_normal_f32(9, 0.3, (K,)) + 1.0)
    ob, (xq, sa) = gpu.norm_linear(dev(x), dev(g), W, B)
    rq, rsa = O.norm_quant(x, g, B)
    rb, _ = O.linear(rq, rsa, p, s, cs, N)
    np.testing.assert_array_equal(host(xq), rq)
    np.testing.assert_array_equal(host(sa), rsa)
    np.testing.assert_array_equal(host(ob), rb)


# ------------------------------------------- one n-tile per workgroup (2..16 rows)
@pytest.mark.parametrize("M", [2, 16])
def test_skinny_one_tile_per_workgroup(gpu, O, tune_env, M):
    tune_env(BQ_SKINNY2=0)
    K, N = 2816, 8224  # 514 tiles
    q, s, W = weight(gpu, O, N, K, 128, seed=46)
    p, cs = O.pack_and_colsum(q)
    x = O.synth_normal_bf16(47, 1.0, (M, K))
    xq, sa = O.norm_quant(x, np.full(K, ONE, np.uint16), 128)
    ob, of = gpu.linear(dev(xq), dev(sa), W, want_f32=True)
    rb, rf = O.linear(xq, sa, p, s, cs, N)
    np.testing.assert_array_equal(host(of), rf)
    np.testing.assert_array_equal(host(ob), rb)


@pytest.mark.parametrize("M", [2, 7, 16])
def test_skinny_tiles_per_workgroup(gpu, O, tune_env, M):
    """q/k/v of 8224/4128/4128 rows (514 + 258 + 258 = 1030 tiles) with 4 (the
    default here), 3, 2 and 1 n-tiles per workgroup: groups straddle segments
    and the last group is short; every segment = the oracle, bit-exact."""
    K = 2816
    x = O.synth_normal_bf16(48 + M, 1.0, (M, K))
    xq, sa = O.norm_quant(x, np.full(K, ONE, np.uint16), 128)
    ws = [weight(gpu, O, n, K, 128, seed=sd) for n, sd in ((8224, 49), (4128, 50), (4128, 51))]
    refs = []
    for q, s, W in ws:
        p, cs = O.pack_and_colsum(q)
        refs.append(O.linear(xq, sa, p, s, cs, W.n_rows)[0])
    for cap in (1, 3, 2, 0):
        tune_env(BQ_SKINNY2=cap)
        outs = gpu.qkv(dev(xq), dev(sa), *(w[2] for w in ws))
        for seg, (o, r) in enumerate(zip(outs, refs)):
            o = host(o)
            bad = np.argwhere(o != r)
            assert bad.size == 0, (cap, seg, bad[:8].tolist(), o[tuple(bad[0])], r[tuple(bad[0])])


# --------------------------------------------------------------- MoE prep forms
@pytest.mark.parametrize("sw", [dict(BQ_MOE_PREP=0), dict(BQ_PREP_ONE=0),
                                dict(BQ_NQ_V8=0)])
@pytest.mark.parametrize("T", [1, 16, 32, 129])
def test_moe_prep_switches(gpu, O, tune_env, sw, T):
    tune_env(**sw)
    E, k, H, B = 128, 8, 2816, 128
    logits = O.synth_normal_f32(70 + T, 1.0, (T, E))
    x = O.synth_normal_bf16(72 + T, 1.0, (T, H))
    g = O.f32_to_bf16(O.synth_normal_f32(73, 0.3, (H,)) + 1.0)
    ridx, rw = O.route_topk_softmax(logits, k, None)
    reo, rroutes = O.build_schedule(ridx, rw, E)
    rq, rsa = O.norm_quant(x, g, B)
    for _ in range(2):
        idx, w, eo, routes, xq, sa = gpu.moe_prep(dev(logits), dev(x), dev(g), k, None, block=B)
        np.testing.assert_array_equal(host(idx), ridx)
        np.testing.assert_array_equal(host(w), rw)
        np.testing.assert_array_equal(host(eo), reo)
        r = host(routes)
        np.testing.assert_array_equal(r[:, 0], rroutes["token"])
        np.testing.assert_array_equal(r[:, 1].view(np.float32), rroutes["weight"])
        np.testing.assert_array_equal(host(xq), rq)
        np.testing.assert_array_equal(host(sa), rsa)
    # bq_ffn_prep under the same switch: the dense norm-quant of the same rows
    gd = O.f32_to_bf16(O.synth_normal_f32(74, 0.3, (H,)) + 1.0)
    rdq, rdsa = O.norm_quant(x, gd, B)
    outs = gpu.ffn_prep(dev(logits), dev(x), dev(g), dev(gd), k, block=B)
    for a, b in zip(outs[:6], (idx, w, eo, routes, xq, sa)):
        np.testing.assert_array_equal(host(a), host(b))
    np.testing.assert_array_equal(host(outs[6]), rdq)
    np.testing.assert_array_equal(host(outs[7]), rdsa)


# ----------------------------------------------------------------- MoE kernels
def _moe_check(gpu, O, T, E=8, k=2, H=256, I=128, seed=5):
    """phase 1 (+ block-quant) and phase 2 on the GPU against the oracle."""
    logits = O.synth_normal_f32(seed, 1.0, (T, E))
    idx, w = O.route_topk_softmax(logits, k)
    gu = O.bf16_to_f32(O.synth_normal_bf16(6, 0.02, (E * 2 * I, H)))
    gq, gs = O.rotate_and_quant(gu, 128)
    dn = O.bf16_to_f32(O.synth_normal_bf16(7, 0.02, (E * H, I)))
    dq, ds = O.rotate_and_quant(dn, 64)
    x = O.synth_normal_bf16(8, 1.0, (T, H))
    xq, xsa = O.norm_quant(x, np.full(H, ONE, np.uint16), 128)
    Wgu = gpu.ButterquantWeight(gpu.retile(dev(gq.reshape(-1)), E * 2 * I, H), dev(gs),
                                E * 2 * I, H)
    Wd = gpu.ButterquantWeight(gpu.retile(dev(dq.reshape(-1)), E * H, I), dev(ds), E * H, I)
    eo, routes = gpu.build_schedule(dev(idx), dev(w), E)
    bi8, bsa, bucket = gpu.moe_phase1_quant(dev(xq), dev(xsa), eo, routes, Wgu, E, T, k, I,
                                            bucket=True)
    accum, out = gpu.moe_phase2(bi8, bsa, eo, routes, Wd, E, T, k, H)
    reo, rroutes = O.build_schedule(idx, w, E)
    gp, gcs = O.pack_and_colsum(gq)
    rb = O.moe_phase1(xq, xsa, reo, rroutes, gp, gs, gcs, I)
    np.testing.assert_array_equal(host(bucket), rb)
    rbq, rbsa = O.block_quant(rb, 64, True)
    np.testing.assert_array_equal(host(bi8), rbq)
    np.testing.assert_array_equal(host(bsa), rbsa)
    dp, dcs = O.pack_and_colsum(dq, 64, False)
    racc, rout = O.moe_phase2(rbq, rbsa, reo, rroutes, T, dp, ds, dcs, H)
    np.testing.assert_array_equal(host(accum), racc)
    np.testing.assert_array_equal(host(out), rout)


@pytest.mark.parametrize("sw", [dict(BQ_DOWN_SKINNY=12), dict(BQ_DOWN_SKINNY=14),
                                dict(BQ_DOWN_SKINNY=21), dict(BQ_DOWN_SKINNY=22),
                                dict(BQ_DOWN_SKINNY=42), dict(BQ_GU_SKINNY=2),
                                dict(BQ_GU_SKINNY=6)])
@pytest.mark.parametrize("T", [5, 40])
def test_moe_skinny_switches(gpu, O, tune_env, sw, T):
    tune_env(**sw)
    _moe_check(gpu, O, T)
    _ffn_check(gpu, O, T)


def _ffn_check(gpu, O, T, E=8, k=2, H=256, I=128, DI=192):
    """bq_ffn_gate_up / bq_ffn_down: the experts' outputs equal the separate
    MoE calls', the dense MLP's the oracle chain's (the dense rows ride in
    the same skinny kernels, so every variant of them is checked)."""
    idx, w = O.route_topk_softmax(O.synth_normal_f32(T + 9, 1.0, (T, E)), k)
    _, _, Wgu = weight(gpu, O, E * 2 * I, H, 128, seed=31)
    _, _, Wd = weight(gpu, O, E * H, I, 64, seed=32)
    ones = np.full(H, ONE, np.uint16)
    xq, xsa = O.norm_quant(O.synth_normal_bf16(T + 10, 1.0, (T, H)), ones, 128)
    dq, dsa = O.norm_quant(O.synth_normal_bf16(T + 11, 1.0, (T, H)), ones, 128)
    (qg, sg, Wg), (qu, su, Wu) = (weight(gpu, O, DI, H, 128, seed=sd) for sd in (33, 34))
    qd, sd, Wdd = weight(gpu, O, H, DI, 64, seed=35)
    rdq, rdsa = _dense_gate_up_ref(O, dq, dsa, qg, sg, qu, su, DI)
    pd, cd = O.pack_and_colsum(qd, 64, False)
    rdo, _ = O.block_linear(rdq, rdsa, pd, sd, cd, H, 64)
    eo, routes = gpu.build_schedule(dev(idx), dev(w), E)
    mi8, msa = gpu.moe_phase1_quant(dev(xq), dev(xsa), eo, routes, Wgu, E, T, k, I)
    macc, mout = gpu.moe_phase2(mi8, msa, eo, routes, Wd, E, T, k, H)
    bi8, bsa, di8, dsa_ = gpu.ffn_gate_up(dev(xq), dev(xsa), eo, routes, Wgu, E, T, k, I,
                                          dev(dq), dev(dsa), Wg, Wu)
    acc, out, do = gpu.ffn_down(bi8, bsa, eo, routes, Wd, E, T, k, H, di8, dsa_, Wdd)
    for a, b in ((bi8, mi8), (bsa, msa), (acc, macc), (out, mout)):
        np.testing.assert_array_equal(host(a), host(b))
    np.testing.assert_array_equal(host(di8), rdq)
    np.testing.assert_array_equal(host(dsa_), rdsa)
    np.testing.assert_array_equal(host(do), rdo)


@pytest.mark.parametrize("sw", [dict(BQ_MOE_ORDER=1), dict(BQ_MOE_ORDER=2),
                                dict(BQ_MOE_ORDER=2, BQ_DOWN_BREG=0),
                                dict(BQ_RING=3), dict(BQ_RING=4), dict(BQ_RING=6),
                                dict(BQ_DOWN_BREG=0, BQ_MOE_BM_DOWN=128),
                                dict(BQ_DOWN_BREG=0, BQ_MOE_BM_DOWN=192),
                                dict(BQ_DOWN_BREG=0, BQ_MOE_BM_DOWN=256)])
@pytest.mark.parametrize("T", [300, 700])
def test_moe_tiled_switches(gpu, O, tune_env, sw, T):
    tune_env(**sw)
    _moe_check(gpu, O, T)


@pytest.mark.parametrize("sw", [dict(BQ_RING=2), dict(BQ_RING=4), dict(BQ_TILE_KSP=1)])
@pytest.mark.parametrize("M,K", [(512, 4096), (200, 2816)])
def test_dense_tiled_switches(gpu, O, tune_env, sw, M, K):
    tune_env(**sw)
    N = 256
    q, s, W = weight(gpu, O, N, K, 128)
    p, cs = O.pack_and_colsum(q)
    x = O.synth_normal_bf16(1, 1.0, (M, K))
    xq, sa = O.norm_quant(x, np.full(K, ONE, np.uint16), 128)
    ob = gpu.linear(dev(xq), dev(sa), W)
    rb, _ = O.linear(xq, sa, p, s, cs, N)
    np.testing.assert_array_equal(host(ob), rb)


# ------------------------------------------------------------- vocabulary head
@pytest.mark.parametrize("sw", [dict(BQ_SEL_FUSED=0), dict(BQ_HEAD_GRID=16),
                                dict(BQ_HEAD_GRID=37), dict(BQ_NQ_V8=0)])
@pytest.mark.parametrize("R", [1, 5])
def test_head_switches(gpu, O, tune_env, sw, R):
    from test_gpu_head import check_outcomes, head_inputs, run_sample, upload_head
    tune_env(**sw)
    V, H = 8192, 2816
    xq, xsa, w, ws = head_inputs(O, R, V, H, 50 + R)
    rng = np.random.default_rng(R)
    params = O.sampling_params(
        R, temperature=rng.choice([1.0, 0.7], R), min_p=rng.choice([0.0, 0.05], R),
        top_k=rng.choice([0, 40], R), seed=rng.integers(0, 2 ** 62, R),
        n_keep=rng.choice([256, 20], R), greedy=rng.random(R) < 0.3)
    W = upload_head(gpu, w, ws)
    check_outcomes(run_sample(gpu, O, xq, xsa, W, params), O.flash_sample(xq, xsa, w, ws, params))
    x = O.synth_normal_bf16(40 + R, 1.0, (R, H))
    gm = O.f32_to_bf16(np.linspace(0.5, 1.5, H).astype(np.float32))
    q, sa = gpu.head_prep(dev(x), dev(gm), 128)
    rq, rsa = O.norm_quant(x, gm, 128, per_block=True)
    np.testing.assert_array_equal(host(q), rq)
    np.testing.assert_array_equal(host(sa), rsa)


# ------------------------------------------------------------ attention splits
@pytest.mark.parametrize("waves", [256, 8192])
@pytest.mark.parametrize("name", ["sliding_decode_16", "full_decode_2"])
def test_attention_waves_switch(gpu, O, tune_env, waves, name):
    from attn_cases import make_case
    from test_gpu_attn import SHAPES, check
    tune_env(BQ_ATTN_WAVES=waves)
    c = make_case(O, 21, **SHAPES[name])
    w = SHAPES[name].get("window", 0)
    s_max = gpu.attention_splits(c.T, c.num_kv, w if w else int(c.positions.max()) + 1)
    check(gpu, O, c, s_max)
