"""GPU parity of the LDS-tiled MFMA paths (prefill linears and the grouped MoE
kernels) for every tile height and both MFMA tiles (v_mfma_i32_16x16x64_i8
and v_mfma_i32_32x32x32_i8), against the CPU oracle, bit-exact.  Tile heights
and the MFMA tile are forced through the library's BQ_TILE_BM / BQ_MOE_BM /
BQ_MF switches."""
import numpy as np
import pytest

from test_gpu_parity import dev, host, tol_check

pytestmark = pytest.mark.gpu
ONE = 0x3F80


@pytest.mark.parametrize("mf", [16, 32])
@pytest.mark.parametrize("bn", [64, 128, 256])
@pytest.mark.parametrize("bm", [32, 64, 128])
@pytest.mark.parametrize("M,K,B", [(200, 512, None), (77, 2816, None), (150, 1024, 256),
                                   (96, 704, 64), (130, 2112, 64), (40, 4096, 64)])
def test_dense_tiles(gpu, O, tune_env, bm, bn, mf, M, K, B):
    tune_env(BQ_TILE_BM=bm, BQ_TILE_BN=bn, BQ_MF=mf)
    N = 384  # 1.5 n-tiles at bn=256; N=2816 tails are covered in test_gpu_parity
    wf = O.bf16_to_f32(O.synth_normal_bf16(3, 0.02, (N, K)))
    q, s = O.rotate_and_quant(wf, B or 128)
    W = gpu.ButterquantWeight(gpu.retile(dev(q.reshape(-1)), N, K), dev(s), N, K)
    x = O.synth_normal_bf16(4, 1.0, (M, K))
    if B is None:
        xq, sa = O.norm_quant(x, np.full(K, ONE, np.uint16), 128 if K % 128 == 0 else 64)
        ob, of = gpu.linear(dev(xq), dev(sa), W, want_f32=True)
        p, cs = O.pack_and_colsum(q)
        rb, rf = O.linear(xq, sa, p, s, cs, N)
    else:
        xq, sa = O.block_quant(x, B, B == 64)
        ob, of = gpu.block_linear(dev(xq), dev(sa), W, B, want_f32=True)
        p, cs = O.pack_and_colsum(q, B, False)
        rb, rf = O.block_linear(xq, sa, p, s, cs, N, B)
    np.testing.assert_array_equal(host(of), rf)
    np.testing.assert_array_equal(host(ob), rb)


@pytest.mark.parametrize("mf", [16, 32])
@pytest.mark.parametrize("M,K,N", [(200, 512, 384), (77, 2816, 384), (512, 4096, 4096),
                                   (64, 128, 256), (130, 704, 256), (33, 192, 128)])
def test_dense_split_k(gpu, O, tune_env, mf, M, K, N):
    # per-row 64 x 128 tiles with two K groups per workgroup (odd, even and
    # single-stage K: the groups get equal stage counts, one more, or none)
    tune_env(BQ_TILE_BM=64, BQ_TILE_BN=128, BQ_TILE_KSP=2, BQ_MF=mf)
    wf = O.bf16_to_f32(O.synth_normal_bf16(3, 0.02, (N, K)))
    q, s = O.rotate_and_quant(wf, 64)
    W = gpu.ButterquantWeight(gpu.retile(dev(q.reshape(-1)), N, K), dev(s), N, K)
    x = O.synth_normal_bf16(4, 1.0, (M, K))
    xq, sa = O.norm_quant(x, np.full(K, ONE, np.uint16), 64)
    ob, of = gpu.linear(dev(xq), dev(sa), W, want_f32=True)
    p, cs = O.pack_and_colsum(q)
    rb, rf = O.linear(xq, sa, p, s, cs, N)
    np.testing.assert_array_equal(host(of), rf)
    np.testing.assert_array_equal(host(ob), rb)


def test_dense_qkv_tiled(gpu, O):
    K, M = 512, 100
    Ws, qs = [], []
    for n, seed in ((256, 1), (128, 2), (128, 3)):
        wf = O.bf16_to_f32(O.synth_normal_bf16(seed, 0.02, (n, K)))
        q, s = O.rotate_and_quant(wf, 128)
        Ws.append(gpu.ButterquantWeight(gpu.retile(dev(q.reshape(-1)), n, K), dev(s), n, K))
    x = O.synth_normal_bf16(6, 1.0, (M, K))
    xq, sa = O.norm_quant(x, np.full(K, ONE, np.uint16), 128)
    outs = gpu.qkv(dev(xq), dev(sa), *Ws)
    for o, W in zip(outs, Ws):
        np.testing.assert_array_equal(host(o), host(gpu.linear(dev(xq), dev(sa), W)))


def _tiny_moe(O, gpu, T, E=4, k=2, H=128, I=64, seed=5):
    logits = O.synth_normal_f32(seed, 1.0, (T, E))
    idx, w = O.route_topk_softmax(logits, k)
    gu = O.bf16_to_f32(O.synth_normal_bf16(6, 0.02, (E * 2 * I, H)))
    gq, gs = O.rotate_and_quant(gu, 128)
    dn = O.bf16_to_f32(O.synth_normal_bf16(7, 0.02, (E * H, I)))
    dq, ds = O.rotate_and_quant(dn, 64)
    x = O.synth_normal_bf16(8, 1.0, (T, H))
    xq, xsa = O.norm_quant(x, np.full(H, ONE, np.uint16), 128)
    Wgu = gpu.ButterquantWeight(gpu.retile(dev(gq.reshape(-1)), E * 2 * I, H), dev(gs), E * 2 * I, H)
    Wd = gpu.ButterquantWeight(gpu.retile(dev(dq.reshape(-1)), E * H, I), dev(ds), E * H, I)
    return dict(idx=idx, w=w, gq=gq, gs=gs, dq=dq, ds=ds, xq=xq, xsa=xsa, Wgu=Wgu, Wd=Wd,
                T=T, E=E, k=k, H=H, I=I)


@pytest.mark.parametrize("T,bm,bn", [(64, None, None), (256, None, None), (64, 128, None),
                                     (256, 64, None), (256, 16, None), (300, 128, None),
                                     (33, 64, None), (256, 128, 128), (256, 64, 64),
                                     (300, 128, 256), (300, 64, 256), (300, 256, None),
                                     (64, 256, None), (600, 256, None), (600, 256, 256),
                                     (300, 256, 256), (300, 192, None), (600, 192, 256),
                                     (600, 192, 128), (64, 192, None)])
@pytest.mark.parametrize("mf", [16, 32])
def test_moe_tiled(gpu, O, tune_env, T, bm, bn, mf):
    tune_env(BQ_MF=mf)
    if bm is not None:
        tune_env(BQ_MOE_BM=bm)
    if bn is not None:
        tune_env(BQ_TILE_BN=bn)
    c = _tiny_moe(O, gpu, T)
    E, H, I, k = c["E"], c["H"], c["I"], c["k"]
    eo, routes = gpu.build_schedule(dev(c["idx"]), dev(c["w"]), E)
    bucket = gpu.moe_phase1(dev(c["xq"]), dev(c["xsa"]), eo, routes, c["Wgu"], E, T, k, I)
    bi8, bsa = gpu.block_quant(bucket, 64, True)
    accum, out = gpu.moe_phase2(bi8, bsa, eo, routes, c["Wd"], E, T, k, H)
    reo, rroutes = O.build_schedule(c["idx"], c["w"], E)
    gp, gcs = O.pack_and_colsum(c["gq"])
    rb = O.moe_phase1(c["xq"], c["xsa"], reo, rroutes, gp, c["gs"], gcs, I)
    np.testing.assert_array_equal(host(bucket), rb)
    rbq, rbsa = O.block_quant(rb, 64, True)
    dp, dcs = O.pack_and_colsum(c["dq"], 64, False)
    racc, rout = O.moe_phase2(rbq, rbsa, reo, rroutes, T, dp, c["ds"], dcs, H)
    np.testing.assert_array_equal(host(accum), racc)
    np.testing.assert_array_equal(host(out), rout)
    tol_check(host(accum), racc)


@pytest.mark.parametrize("T", [600, 512])
def test_moe_gate_up_hidden2816(gpu, O, T):
    # model hidden size (K/64 = 44) with ~150 (T = 600: 256-record tiles) or
    # ~128 (T = 512: 192-record tiles) routes per expert: partial m-tiles and a
    # partial gate/up n-tile (inter 192)
    E, k, H, I = 8, 2, 2816, 192
    logits = O.synth_normal_f32(21, 1.0, (T, E))
    idx, w = O.route_topk_softmax(logits, k)
    gu = O.bf16_to_f32(O.synth_normal_bf16(22, 0.02, (E * 2 * I, H)))
    gq, gs = O.rotate_and_quant(gu, 128)
    x = O.synth_normal_bf16(23, 1.0, (T, H))
    xq, xsa = O.norm_quant(x, np.full(H, ONE, np.uint16), 128)
    Wgu = gpu.ButterquantWeight(gpu.retile(dev(gq.reshape(-1)), E * 2 * I, H), dev(gs), E * 2 * I, H)
    eo, routes = gpu.build_schedule(dev(idx), dev(w), E)
    bucket = gpu.moe_phase1(dev(xq), dev(xsa), eo, routes, Wgu, E, T, k, I)
    reo, rroutes = O.build_schedule(idx, w, E)
    gp, gcs = O.pack_and_colsum(gq)
    rb = O.moe_phase1(xq, xsa, reo, rroutes, gp, gs, gcs, I)
    np.testing.assert_array_equal(host(bucket), rb)


@pytest.mark.parametrize("T,breg,mf", [(64, "0", 16), (300, "0", 16), (600, "0", 16),
                                       (64, "0", 32), (300, "0", 32), (600, "0", 32),
                                       (33, "1", 32), (300, "1", 32)])
def test_moe_down_paths(gpu, O, tune_env, T, breg, mf):
    # the down projection with weights in registers (default for block 64 and
    # inter <= 704) and the LDS-ring k_tiled path it replaces
    tune_env(BQ_DOWN_BREG=breg, BQ_MF=mf)
    c = _tiny_moe(O, gpu, T)
    E, H, I, k = c["E"], c["H"], c["I"], c["k"]
    eo, routes = gpu.build_schedule(dev(c["idx"]), dev(c["w"]), E)
    reo, rroutes = O.build_schedule(c["idx"], c["w"], E)
    gp, gcs = O.pack_and_colsum(c["gq"])
    rb = O.moe_phase1(c["xq"], c["xsa"], reo, rroutes, gp, c["gs"], gcs, I)
    rbq, rbsa = O.block_quant(rb, 64, True)
    accum, out = gpu.moe_phase2(dev(rbq), dev(rbsa), eo, routes, c["Wd"], E, T, k, H)
    dp, dcs = O.pack_and_colsum(c["dq"], 64, False)
    racc, rout = O.moe_phase2(rbq, rbsa, reo, rroutes, T, dp, c["ds"], dcs, H)
    np.testing.assert_array_equal(host(accum), racc)
    np.testing.assert_array_equal(host(out), rout)


@pytest.mark.parametrize("T", [450, 200, 130, 20])
def test_moe_down_hidden2816(gpu, O, T):
    # model shapes (hidden 2816 = 11 column tiles of 256, inter 704 = 11
    # k-steps): T = 450 gives ~225 records per expert (a full and a partial
    # 192-record m-tile), T = 200 one partial m-tile, T = 130 ~65 records,
    # T = 20 ~10 records (the skinny 16-record kernel)
    E, k, H, I = 4, 2, 2816, 704
    rng = np.random.default_rng(T)
    logits = O.synth_normal_f32(31, 1.0, (T, E))
    idx, w = O.route_topk_softmax(logits, k)
    dn = O.bf16_to_f32(O.synth_normal_bf16(32, 0.02, (E * H, I)))
    dq, ds = O.rotate_and_quant(dn, 64)
    Wd = gpu.ButterquantWeight(gpu.retile(dev(dq.reshape(-1)), E * H, I), dev(ds), E * H, I)
    bucket = O.f32_to_bf16(rng.standard_normal((T * k, I)).astype(np.float32))
    bq, bsa = O.block_quant(bucket, 64, True)
    eo, routes = gpu.build_schedule(dev(idx), dev(w), E)
    print(f"moe down H={H} I={I} T={T}", flush=True)
    accum, out = gpu.moe_phase2(dev(bq), dev(bsa), eo, routes, Wd, E, T, k, H)
    reo, rroutes = O.build_schedule(idx, w, E)
    dp, dcs = O.pack_and_colsum(dq, 64, False)
    racc, rout = O.moe_phase2(bq, bsa, reo, rroutes, T, dp, ds, dcs, H)
    np.testing.assert_array_equal(host(accum), racc)
    np.testing.assert_array_equal(host(out), rout)
