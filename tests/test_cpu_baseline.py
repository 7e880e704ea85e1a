"""The CPU baseline (oracle/cpu_baseline.c: the reference's VNNI branch with
vpdpbusd, 32-row tiles over worker_range and the reference's worker policies)
against the scalar oracle (oracle/bq_oracle.c), bit for bit, on small shapes
and several thread counts.

This makes the port that bench.py times a verified restatement of the
reference CPU path, and lets GPU tests use it as a fast full-size checker.
Every compared output is the reference's own bf16 / f32 / int8 result, so a
slip in the port's tile walk, colsum correction, drain order or worker split
fails here."""
import numpy as np
import pytest

ONE = 0x3F80


@pytest.fixture(scope="module")
def vnni(O):
    isa = O.cpu().bqcpu_isa().decode()
    if isa != "avx512vnni":
        pytest.skip(f"host has no AVX-512 VNNI ({isa}): the port would only call the oracle")
    return O


def weights(O, n, k, block, seed, per_block_cs=False):
    w = O.bf16_to_f32(O.synth_normal_bf16(seed, 0.02, (n, k)))
    q, s = O.rotate_and_quant(w, block)
    p, cs = O.pack_and_colsum(q, block, False) if per_block_cs else O.pack_and_colsum(q)
    return q, s, p, cs


@pytest.mark.parametrize("M,K,threads", [(1, 256, 1), (1, 2816, 3), (5, 2816, 8), (17, 512, 5)])
def test_cpu_linear(vnni, M, K, threads):
    O = vnni
    N = 256
    _, s, p, cs = weights(O, N, K, 128, 0)
    xq, sa = O.norm_quant(O.synth_normal_bf16(1, 1.0, (M, K)), np.full(K, ONE, np.uint16), 128)
    rb, _ = O.linear(xq, sa, p, s, cs, N)
    np.testing.assert_array_equal(O.cpu_linear(xq, sa, p, s, cs, N, threads), rb)


@pytest.mark.parametrize("M,K,B,threads", [(1, 2112, 64, 4), (6, 1024, 256, 3), (9, 2048, 512, 8)])
def test_cpu_block_linear(vnni, M, K, B, threads):
    O = vnni
    N = 128
    _, s, p, cs = weights(O, N, K, B, 4, per_block_cs=True)
    xq, sa = O.block_quant(O.synth_normal_bf16(5, 1.0, (M, K)), B, B == 64)
    rb, _ = O.block_linear(xq, sa, p, s, cs, N, B)
    np.testing.assert_array_equal(O.cpu_block_linear(xq, sa, p, s, cs, N, B, threads), rb)


@pytest.mark.parametrize("T,H,threads", [(3, 2816, 2), (40, 2816, 8), (33, 512, 3)])
def test_cpu_norm_quant(vnni, T, H, threads):
    O = vnni
    x = O.synth_normal_bf16(11, 1.0, (T, H))
    g = O.f32_to_bf16(O.synth_normal_f32(12, 0.3, (H,)) + 1.0)
    q, sa = O.cpu_norm_quant(x, g, 128, threads)
    rq, rsa = O.norm_quant(x, g, 128)
    np.testing.assert_array_equal(sa, rsa)
    np.testing.assert_array_equal(q, rq)


@pytest.mark.parametrize("rows,cols,B,fwht", [(50, 704, 64, True), (20, 4096, 256, False)])
def test_cpu_block_quant(vnni, rows, cols, B, fwht):
    O = vnni
    x = O.synth_normal_bf16(2, 1.0, (rows, cols))
    q, sa = O.cpu_block_quant(x, B, fwht, 5)
    rq, rsa = O.block_quant(x, B, fwht)
    np.testing.assert_array_equal(sa, rsa)
    np.testing.assert_array_equal(q, rq)


@pytest.mark.parametrize("T,threads", [(7, 3), (300, 8)])
def test_cpu_route_topk(vnni, T, threads):
    O = vnni
    lg = O.synth_normal_f32(2, 1.0, (T, 128))
    pes = O.f32_to_bf16(O.synth_normal_f32(3, 0.1, (128,)) + 1.0)
    idx, w = O.cpu_route_topk(lg, 8, pes, threads)
    ridx, rw = O.route_topk_softmax(lg, 8, pes)
    np.testing.assert_array_equal(idx, ridx)
    np.testing.assert_array_equal(w, rw)


def small_moe(O, E=16, H=512, I=192, seed=0):
    rng = np.random.default_rng(seed)
    gu = O.bf16_to_f32(O.f32_to_bf16(rng.standard_normal((E * 2 * I, H), np.float32) * np.float32(0.02)))
    gq, gs = O.rotate_and_quant(gu, 128)
    dn = O.bf16_to_f32(O.f32_to_bf16(rng.standard_normal((E * H, I), np.float32) * np.float32(0.02)))
    dq, ds = O.rotate_and_quant(dn, 64)
    gp, gcs = O.pack_and_colsum(gq)
    dp, dcs = O.pack_and_colsum(dq, 64, False)
    return gs, gp, gcs, ds, dp, dcs


@pytest.mark.parametrize("T,threads", [(5, 3), (40, 8)])
def test_cpu_moe_phases(vnni, T, threads):
    O = vnni
    E, H, I = 16, 512, 192
    gs, gp, gcs, ds, dp, dcs = small_moe(O, E, H, I)
    x = O.synth_normal_bf16(1, 1.0, (T, H))
    xq, xsa = O.norm_quant(x, np.full(H, ONE, np.uint16), 128)
    idx, w = O.route_topk_softmax(O.synth_normal_f32(2, 1.0, (T, E)), 8)
    eo, routes = O.build_schedule(idx, w, E)
    rb = O.moe_phase1(xq, xsa, eo, routes, gp, gs, gcs, I)
    np.testing.assert_array_equal(O.cpu_moe_phase1(xq, xsa, eo, routes, gp, gs, gcs, I, threads), rb)
    bq, bsa = O.block_quant(rb, 64, True)
    racc, rout = O.moe_phase2(bq, bsa, eo, routes, T, dp, ds, dcs, H)
    acc, out = O.cpu_moe_phase2(bq, bsa, eo, routes, T, dp, ds, dcs, H, 64, threads)
    np.testing.assert_array_equal(acc, racc)
    np.testing.assert_array_equal(out, rout)


def test_cpu_moe_layer(vnni):
    """bqcpu_moe_layer (the timed CPU layer) equals the oracle's pipeline."""
    O = vnni
    E, H, I, T, k = 16, 512, 192, 24, 8
    gs, gp, gcs, ds, dp, dcs = small_moe(O, E, H, I, seed=1)
    x = O.synth_normal_bf16(1, 1.0, (T, H))
    lg = O.synth_normal_f32(2, 1.0, (T, E))
    g = np.full(H, ONE, np.uint16)
    layer = O.CpuMoeLayer(T, E, k, H, I, gp, gs, gcs, dp, ds, dcs)
    acc, out = layer(lg, x, g, nthreads=6)
    idx, w = O.route_topk_softmax(lg, k)
    eo, routes = O.build_schedule(idx, w, E)
    xq, xsa = O.norm_quant(x, g, 128)
    b = O.moe_phase1(xq, xsa, eo, routes, gp, gs, gcs, I)
    bq, bsa = O.block_quant(b, 64, True)
    racc, rout = O.moe_phase2(bq, bsa, eo, routes, T, dp, ds, dcs, H)
    np.testing.assert_array_equal(layer.eo, eo)
    np.testing.assert_array_equal(acc, racc)
    np.testing.assert_array_equal(out, rout)


def test_worker_policy_pin(vnni):
    """Pinning the OpenMP team succeeds on the CPUs this process may use."""
    import os
    orig = os.sched_getaffinity(0)
    cpus = sorted(orig)[:2]
    try:
        vnni.cpu_pin(cpus)
        assert os.sched_getaffinity(0) == {cpus[0]}  # the calling thread is thread 0
    finally:
        os.sched_setaffinity(0, orig)
