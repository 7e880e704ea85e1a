"""GPU parity: libbq.so (through its C ABI) against the CPU oracle and the
committed fixtures, on identical seeded inputs.

Bar (tolerances are stated per assertion):
  * int8 codes, re-tiled/unpacked bytes, colsums, schedules: bit-exact;
  * f32 outputs of the linears and the MoE: bit-exact with the oracle's
    signed-form restatement (which equals the reference's VNNI u8/colsum
    form whenever |sum (x+128)w| < 2^24, asserted where it matters); the
    floating-point tolerance (normwise rel 1e-3, cosine > 0.9999) is checked too.
"""
import os

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "golden.npz")
ONE = 0x3F80


# ---------------------------------------------------------------- helpers
def dev(a):
    import torch
    a = np.ascontiguousarray(a)
    if a.dtype == np.uint16:
        return torch.from_numpy(a.view(np.int16)).cuda().view(torch.bfloat16)
    return torch.from_numpy(a).cuda()


def host(t):
    import torch
    if t.dtype == torch.bfloat16:
        return t.view(torch.int16).cpu().numpy().view(np.uint16)
    return t.cpu().numpy()


def tol_check(got, ref):
    got = np.asarray(got, np.float64).ravel()
    ref = np.asarray(ref, np.float64).ravel()
    rel = np.abs(got - ref).max() / max(np.abs(ref).max(), 1e-30)
    cos = got @ ref / (np.linalg.norm(got) * np.linalg.norm(ref) + 1e-300)
    assert rel <= 1e-3 and cos > 0.9999, (rel, cos)


def weight(gpu, O, n, k, block, seed=0):
    """Quantize with the oracle (reference recipe), upload, re-tile on GPU."""
    wf = O.bf16_to_f32(O.synth_normal_bf16(seed, 0.02, (n, k)))
    q, s = O.rotate_and_quant(wf, block)
    t = gpu.retile(dev(q.reshape(-1)), n, k)
    return q, s, gpu.ButterquantWeight(t, dev(s), n, k)


@pytest.fixture(scope="module")
def G():
    return dict(np.load(GOLDEN, allow_pickle=False))


# ---------------------------------------------------------------- layout
def test_retile_unpack_roundtrip(gpu):
    rng = np.random.default_rng(0)
    n, k = 96, 320
    w = rng.integers(-128, 128, (n, k), dtype=np.int8)
    t = gpu.retile(dev(w.reshape(-1)), n, k)
    th = host(t)
    # tile16x64 definition: fragment (n/16, k/64), lane ((k%64)/16)*16 + n%16
    nn, kk = np.meshgrid(np.arange(n), np.arange(k), indexing="ij")
    off = ((nn // 16) * (k // 64) + kk // 64) * 1024 + (((kk % 64) // 16) * 16 + nn % 16) * 16 + kk % 16
    np.testing.assert_array_equal(th[off], w)
    np.testing.assert_array_equal(host(gpu.unpack(t, n, k)), w)


def test_retile_from_reference_vnni(gpu, O):
    rng = np.random.default_rng(1)
    n, k = 64, 256
    w = rng.integers(-128, 128, (n, k), dtype=np.int8)
    p, _ = O.pack_and_colsum(w)
    a = gpu.retile(dev(p), n, k, gpu.LAYOUT_VNNI)
    b = gpu.retile(dev(w.reshape(-1)), n, k)
    np.testing.assert_array_equal(host(a), host(b))


@pytest.mark.parametrize("block,row_major", [(None, True), (64, False), (16, True)])
def test_pack_colsum_vnni(gpu, O, G, block, row_major):
    w = G["pack_w"]
    p, cs = gpu.pack_colsum_vnni(dev(w), block, row_major)
    rp, rcs = O.pack_and_colsum(w, block, row_major)
    np.testing.assert_array_equal(host(p), rp)
    np.testing.assert_array_equal(host(cs), rcs)
    if block is None:
        np.testing.assert_array_equal(host(p), G["pack_vnni"])
        np.testing.assert_array_equal(host(cs), G["pack_colsum"])


@pytest.mark.parametrize("B,per_block", [(128, False), (64, False), (16, False), (256, False),
                                         (512, False), (64, True), (32, True)])
def test_quantize_weight(gpu, O, B, per_block):
    n, k = 48, 1024
    w = O.synth_normal_bf16(0, 0.02, (n, k))
    q, s = gpu.quantize_weight(dev(w), B, per_block)
    rq, rs = O.rotate_and_quant(O.bf16_to_f32(w), B, per_block)
    np.testing.assert_array_equal(host(q), rq)
    np.testing.assert_array_equal(host(s), rs)


def test_quantize_weight_golden(gpu, G):
    q, s = gpu.quantize_weight(dev(G["rq_w"]), 128)
    np.testing.assert_array_equal(host(q), G["rq_codes"])
    np.testing.assert_array_equal(host(s), G["rq_scales"])
    q, s = gpu.quantize_weight(dev(G["rq_w"]), 64, True)
    np.testing.assert_array_equal(host(q), G["rq_codes_pb64"])
    np.testing.assert_array_equal(host(s), G["rq_scales_pb64"])


# ---------------------------------------------------------------- activations
@pytest.mark.parametrize("H,B", [(2816, 128), (4096, 128), (2112, 64), (512, 16), (4096, 512),
                                 (1024, 32), (8192, 256), (2048, 512), (2048, 128), (3072, 256),
                                 (3072, 128), (1024, 512), (256, 128), (2304, 256), (3584, 64)])
def test_norm_quant(gpu, O, H, B):
    # few tokens: a token's segments spread over up to 8 waves (whole FWHT
    # blocks per wave, 1 to 4 segments of 128 values each)
    x = O.synth_normal_bf16(1, 1.0, (5, H))
    g = O.f32_to_bf16(O.synth_normal_f32(9, 0.3, (H,)) + 1.0)
    q, sa = gpu.norm_quant(dev(x), dev(g), B)
    rq, rsa = O.norm_quant(x, g, B)
    np.testing.assert_array_equal(host(sa), rsa)
    np.testing.assert_array_equal(host(q), rq)


@pytest.mark.parametrize("T", [259, 1795])
@pytest.mark.parametrize("H,B", [(2816, 128), (4096, 128), (2112, 64), (512, 16), (4096, 512),
                                 (1024, 32), (768, 256), (1536, 512)])
def test_norm_quant_long(gpu, O, H, B, T):
    # seq_len >= 1792 takes the one-wave-per-token kernel (1795 leaves a
    # partial workgroup); 259 runs the workgroup-per-row kernel on many rows
    x = O.synth_normal_bf16(11, 1.0, (T, H))
    g = O.f32_to_bf16(O.synth_normal_f32(12, 0.3, (H,)) + 1.0)
    q, sa = gpu.norm_quant(dev(x), dev(g), B)
    rq, rsa = O.norm_quant(x, g, B)
    np.testing.assert_array_equal(host(sa), rsa)
    np.testing.assert_array_equal(host(q), rq)


def test_norm_quant_golden(gpu, G):
    q, sa = gpu.norm_quant(dev(G["nq_x"]), dev(G["nq_gamma"]), 128)
    np.testing.assert_array_equal(host(q), G["nq_codes"])
    np.testing.assert_array_equal(host(sa), G["nq_sa"])


def test_norm_quant_zero_row(gpu, O):
    x = np.zeros((2, 256), np.uint16)
    x[1] = O.synth_normal_bf16(3, 1.0, (256,))
    q, sa = gpu.norm_quant(dev(x), dev(np.full(256, ONE, np.uint16)), 128)
    assert host(sa)[0] == 0.0 and (host(q)[0] == 0).all()
    rq, rsa = O.norm_quant(x, np.full(256, ONE, np.uint16), 128)
    np.testing.assert_array_equal(host(q), rq)


@pytest.mark.parametrize("cols,B,fwht", [(704, 64, True), (2112, 64, True), (4096, 256, False),
                                         (8192, 512, False), (512, 16, True), (512, 32, False),
                                         (1024, 128, True)])
def test_block_quant(gpu, O, cols, B, fwht):
    x = O.synth_normal_bf16(2, 1.0, (37, cols))
    q, sa = gpu.block_quant(dev(x), B, fwht)
    rq, rsa = O.block_quant(x, B, fwht)
    np.testing.assert_array_equal(host(sa), rsa)
    np.testing.assert_array_equal(host(q), rq)


@pytest.mark.parametrize("B", [16, 32, 64, 128, 256, 512])
@pytest.mark.parametrize("fwht", [True, False])
def test_block_quant_blocks(gpu, O, B, fwht):
    # every block size of the flat kernel; 3 rows x 1024 columns, plus zero blocks
    x = O.synth_normal_bf16(5, 1.0, (3, 1024))
    x[1, :B] = 0
    q, sa = gpu.block_quant(dev(x), B, fwht)
    rq, rsa = O.block_quant(x, B, fwht)
    assert rsa.reshape(-1)[1024 // B] == 0.0
    np.testing.assert_array_equal(host(sa), rsa)
    np.testing.assert_array_equal(host(q), rq)


@pytest.mark.parametrize("cols,B,fwht", [(704, 64, True), (2048, 256, False)])
def test_block_quant_large(gpu, O, cols, B, fwht):
    # 4001 rows (the 2048-token MoE bucket's scale): 1375+ workgroups, the last partial
    x = O.synth_normal_bf16(5, 1.0, (4001, cols))
    q, sa = gpu.block_quant(dev(x), B, fwht)
    rq, rsa = O.block_quant(x, B, fwht)
    np.testing.assert_array_equal(host(sa), rsa)
    np.testing.assert_array_equal(host(q), rq)


def test_block_quant_golden(gpu, G):
    q, sa = gpu.block_quant(dev(G["bq_x"]), 64, True)
    np.testing.assert_array_equal(host(q), G["bq_codes"])
    np.testing.assert_array_equal(host(sa), G["bq_sa"])


# ---------------------------------------------------------------- linears
@pytest.mark.parametrize("M,K", [(1, 256), (1, 2816), (2, 2816), (16, 2816), (17, 256),
                                 (40, 512), (128, 256), (300, 256), (3, 8192), (16, 6144),
                                 (16, 12288)])
def test_linear(gpu, O, M, K):
    N = 256
    q, s, W = weight(gpu, O, N, K, 128)
    p, cs = O.pack_and_colsum(q)
    x = O.synth_normal_bf16(1, 1.0, (M, K))
    xq, sa = O.norm_quant(x, np.full(K, ONE, np.uint16), 128)
    ob, of = gpu.linear(dev(xq), dev(sa), W, want_f32=True)
    rb, rf = O.linear(xq, sa, p, s, cs, N)          # reference VNNI (u8, colsum) form
    assert np.abs((xq.astype(np.int64) + 128) @ q.astype(np.int64).T).max() < 2 ** 24
    np.testing.assert_array_equal(host(of), rf)
    np.testing.assert_array_equal(host(ob), rb)
    tol_check(host(of), rf)


def test_linear_golden(gpu, G):
    W = gpu.ButterquantWeight(gpu.retile(dev(G["rq_codes"].reshape(-1)), 64, 256),
                              dev(G["rq_scales"]), 64, 256)
    ob, of = gpu.linear(dev(G["lin_xq"]), dev(G["lin_sa"]), W, want_f32=True)
    np.testing.assert_array_equal(host(of), G["lin_out_f32"])
    np.testing.assert_array_equal(host(ob), G["lin_out_bf16"])


@pytest.mark.parametrize("M,K,B", [(1, 2112, 64), (3, 4096, 256), (16, 8192, 512), (5, 8192, 128),
                                   (17, 2112, 64), (33, 1024, 256), (100, 1024, 512),
                                   (64, 704, 64)])
def test_block_linear(gpu, O, M, K, B):
    N = 128
    q, s, W = weight(gpu, O, N, K, B, seed=4)
    p, cs = O.pack_and_colsum(q, B, False)
    x = O.synth_normal_bf16(5, 1.0, (M, K))
    xq, sa = O.block_quant(x, B, B == 64)
    ob, of = gpu.block_linear(dev(xq), dev(sa), W, B, want_f32=True)
    rb, rf = O.block_linear(xq, sa, p, s, cs, N, B)
    np.testing.assert_array_equal(host(of), rf)
    np.testing.assert_array_equal(host(ob), rb)


def test_block_linear_golden(gpu, G):
    W = gpu.ButterquantWeight(gpu.retile(dev(G["blin_codes"].reshape(-1)), 64, 256),
                              dev(G["blin_scales"]), 64, 256)
    ob, of = gpu.block_linear(dev(G["blin_xq"]), dev(G["blin_sa"]), W, 64, want_f32=True)
    np.testing.assert_array_equal(host(of), G["blin_out_f32"])
    np.testing.assert_array_equal(host(ob), G["blin_out_bf16"])


@pytest.mark.parametrize("M", [1, 20])
def test_qkv_matches_three_linears(gpu, O, M):
    K = 512
    Ws = [weight(gpu, O, n, K, 128, seed=s)[2] for n, s in ((256, 1), (128, 2), (128, 3))]
    x = O.synth_normal_bf16(6, 1.0, (M, K))
    xq, sa = O.norm_quant(x, np.full(K, ONE, np.uint16), 128)
    outs = gpu.qkv(dev(xq), dev(sa), *Ws)
    for o, W in zip(outs, Ws):
        np.testing.assert_array_equal(host(o), host(gpu.linear(dev(xq), dev(sa), W)))


@pytest.mark.parametrize("M", [2, 5, 16])
def test_linear_two_tiles(gpu, O, M):
    """2..16 rows with >= 2 n-tiles per CU take two n-tiles per workgroup,
    bit-exact: q/k/v of 4112/2048/2048 rows (257 + 128 + 128 tiles: one
    workgroup's pair straddles q and k, the last tile is alone) against the
    three linears alone (each under 512 tiles: one tile per workgroup; the
    oracle's VNNI pack takes no 4112-row weight), and the full layer's q/k
    pair (8192 + 1024 rows) against the oracle."""
    K = 2816
    x = O.synth_normal_bf16(40 + M, 1.0, (M, K))
    xq, sa = O.norm_quant(x, np.full(K, ONE, np.uint16), 128)
    Ws = [weight(gpu, O, n, K, 128, seed=sd)[2] for n, sd in ((4112, 41), (2048, 42), (2048, 43))]
    outs = gpu.qkv(dev(xq), dev(sa), *Ws)
    for o, W in zip(outs, Ws):
        np.testing.assert_array_equal(host(o), host(gpu.linear(dev(xq), dev(sa), W)))
    ws = [weight(gpu, O, n, K, 128, seed=sd) for n, sd in ((8192, 44), (1024, 45))]
    outs = gpu.linear_pair(dev(xq), dev(sa), ws[0][2], ws[1][2])
    for o, (q, s, W) in zip(outs, ws):
        p, cs = O.pack_and_colsum(q)
        rb, _ = O.linear(xq, sa, p, s, cs, W.n_rows)
        np.testing.assert_array_equal(host(o), rb)


@pytest.mark.parametrize("M,K", [(1, 2816), (16, 2816), (17, 512), (300, 1024)])
def test_linear_pair(gpu, O, M, K):
    """gate and up in one launch = the two linears (and the oracle), bit-exact."""
    (q0, s0, W0), (q1, s1, W1) = (weight(gpu, O, n, K, 128, seed=sd)
                                  for n, sd in ((288, 1), (160, 2)))
    x = O.synth_normal_bf16(6, 1.0, (M, K))
    xq, sa = O.norm_quant(x, np.full(K, ONE, np.uint16), 128)
    o0, o1 = gpu.linear_pair(dev(xq), dev(sa), W0, W1)
    for o, q, s, W in ((o0, q0, s0, W0), (o1, q1, s1, W1)):
        np.testing.assert_array_equal(host(o), host(gpu.linear(dev(xq), dev(sa), W)))
        p, cs = O.pack_and_colsum(q)
        rb, _ = O.linear(xq, sa, p, s, cs, W.n_rows)
        np.testing.assert_array_equal(host(o), rb)


@pytest.mark.parametrize("M,K", [(1, 2816), (1, 4096), (3, 2816)])
def test_norm_linear_pair(gpu, O, M, K):
    """norm-quant + gate and up in one call = norm_quant then the two linears."""
    (q0, s0, W0), (q1, s1, W1) = (weight(gpu, O, n, K, 128, seed=sd)
                                  for n, sd in ((2112, 1), (2112, 2)))
    x = O.synth_normal_bf16(7, 1.0, (M, K))
    gamma = O.f32_to_bf16(O.synth_normal_f32(9, 0.3, (K,)) + 1.0)
    (o0, o1), (xq, sa) = gpu.norm_linear_pair(dev(x), dev(gamma), W0, W1, 128)
    rxq, rsa = O.norm_quant(x, gamma, 128)
    np.testing.assert_array_equal(host(xq), rxq)
    np.testing.assert_array_equal(host(sa), rsa)
    for o, q, s, W in ((o0, q0, s0, W0), (o1, q1, s1, W1)):
        p, cs = O.pack_and_colsum(q)
        rb, _ = O.linear(rxq, rsa, p, s, cs, W.n_rows)
        np.testing.assert_array_equal(host(o), rb)


@pytest.mark.parametrize("M,K,N,B", [(1, 2816, 256, 128), (1, 4096, 512, 128), (1, 2816, 128, 256),
                                     (1, 4096, 256, 512), (1, 512, 256, 64), (1, 1024, 128, 512),
                                     (1, 2304, 256, 256), (1, 768, 128, 16), (3, 2816, 256, 128),
                                     (1, 8192, 128, 256), (1, 2112, 128, 64)])
def test_norm_linear(gpu, O, M, K, N, B):
    """The fused norm-quant + linear (one launch for one token of hidden % 256
    == 0 up to 4096, else the two launches) against the oracle's norm-quant and
    linear: codes, amax and both outputs bit-exact."""
    q, s, W = weight(gpu, O, N, K, 128 if K % 128 == 0 else 64, seed=3)
    p, cs = O.pack_and_colsum(q)
    x = O.synth_normal_bf16(7, 1.0, (M, K))
    g = O.f32_to_bf16(O.synth_normal_f32(9, 0.3, (K,)) + 1.0)
    (ob, of), (xq, sa) = gpu.norm_linear(dev(x), dev(g), W, B, want_f32=True)
    rq, rsa = O.norm_quant(x, g, B)
    np.testing.assert_array_equal(host(sa), rsa)
    np.testing.assert_array_equal(host(xq), rq)
    rb, rf = O.linear(rq, rsa, p, s, cs, N)
    np.testing.assert_array_equal(host(of), rf)
    np.testing.assert_array_equal(host(ob), rb)


def test_norm_linear_zero_row(gpu, O):
    """An all-zero token: amax 0, codes 0, outputs 0, as the two calls give."""
    K, N = 2816, 128
    W = weight(gpu, O, N, K, 128, seed=3)[2]
    x = np.zeros((1, K), np.uint16)
    g = np.full(K, ONE, np.uint16)
    ob, (xq, sa) = gpu.norm_linear(dev(x), dev(g), W, 128)
    rq, rsa = O.norm_quant(x, g, 128)
    np.testing.assert_array_equal(host(sa), rsa)
    np.testing.assert_array_equal(host(xq), rq)
    xq2, sa2 = gpu.norm_quant(dev(x), dev(g), 128)
    np.testing.assert_array_equal(host(ob), host(gpu.linear(xq2, sa2, W)))


@pytest.mark.parametrize("M,K,qn,kvn", [(1, 2816, 4096, 2048), (1, 512, 256, 128),
                                        (2, 2816, 256, 128)])
def test_norm_qkv(gpu, O, M, K, qn, kvn):
    """Fused norm-quant + q|k|v (the decoder's attention input at hidden 2816,
    q 4096 / k, v 2048) against bq_norm_quant then bq_qkv: bit-exact."""
    Ws = [weight(gpu, O, n, K, 128, seed=sd)[2] for n, sd in ((qn, 1), (kvn, 2), (kvn, 3))]
    x = O.synth_normal_bf16(8, 1.0, (M, K))
    g = O.f32_to_bf16(O.synth_normal_f32(4, 0.3, (K,)) + 1.0)
    outs, (xq, sa) = gpu.norm_qkv(dev(x), dev(g), *Ws, block=128)
    xq2, sa2 = gpu.norm_quant(dev(x), dev(g), 128)
    np.testing.assert_array_equal(host(xq), host(xq2))
    np.testing.assert_array_equal(host(sa), host(sa2))
    for o, o2 in zip(outs, gpu.qkv(xq2, sa2, *Ws)):
        np.testing.assert_array_equal(host(o), host(o2))


@pytest.mark.parametrize("M", [1, 512])
def test_linear_full_size(gpu, O, M):
    """Config sizes K = N = 4096: all rows against an exact f64 integer matmul
    with the f32 epilogue in the reference's op order, and sampled rows
    against the oracle."""
    N = K = 4096
    q, s, W = weight(gpu, O, N, K, 128)
    x = O.synth_normal_bf16(1, 1.0, (M, K))
    xq, sa = O.norm_quant(x, np.full(K, ONE, np.uint16), 128)
    ob, of = gpu.linear(dev(xq), dev(sa), W, want_f32=True)
    acc = xq.astype(np.float64) @ q.astype(np.float64).T          # exact: |acc| < 2^53
    inv127 = np.float32(1.0) / np.float32(127.0)
    ref = (acc.astype(np.float32) * (sa * inv127)[:, None]) * s[None, :]
    np.testing.assert_array_equal(host(of), ref.astype(np.float32))
    rows = np.unique(np.linspace(0, M - 1, 3).astype(int))
    p, cs = O.pack_and_colsum(q)
    rb, rf = O.linear(xq[rows], sa[rows], p, s, cs, N)
    np.testing.assert_array_equal(host(of)[rows], rf)
    tol_check(host(of), ref)


# ---------------------------------------------------------------- MoE
def route_table(O, T, E=128, k=8, seed=2):
    logits = O.synth_normal_f32(seed, 1.0, (T, E))
    return O.route_topk_softmax(logits, k)


@pytest.mark.parametrize("T", [1, 32, 128, 129, 1500, 2048])
def test_build_schedule(gpu, O, T):
    # up to 1024 slots (T * 8) one workgroup builds it; 129 tokens and more take
    # the per-expert kernel
    idx, w = route_table(O, T)
    eo, routes = gpu.build_schedule(dev(idx), dev(w), 128)
    reo, rroutes = O.build_schedule(idx, w, 128)
    np.testing.assert_array_equal(host(eo), reo)
    r = host(routes)
    np.testing.assert_array_equal(r[:, 0], rroutes["token"])
    np.testing.assert_array_equal(r[:, 1].view(np.float32), rroutes["weight"])


@pytest.mark.parametrize("T,E,k,pes", [(1, 128, 8, False), (5, 128, 8, True), (16, 60, 8, False),
                                      (16, 256, 16, True), (32, 128, 8, True), (8, 60, 8, True),
                                      (8, 256, 16, False), (9, 128, 8, False),
                                      (128, 128, 8, False), (129, 128, 8, True),
                                      (2048, 128, 8, True), (40, 60, 2, False),
                                      (64, 256, 16, True), (300, 8, 2, False),
                                      (1000, 64, 1, False), (200, 128, 4, True)])
def test_route_schedule(gpu, O, T, E, k, pes):
    """the fused route top-k + schedule equals the two calls and the oracle:
    one workgroup up to 8 tokens (E <= 64, <= 128, <= 256 instances), the
    two kernels above"""
    logits = O.synth_normal_f32(7 + T, 1.0, (T, E))
    sc = O.f32_to_bf16(O.synth_normal_f32(8, 0.2, (E,)) + 1.0) if pes else None
    idx, w, eo, routes = gpu.route_schedule(dev(logits), k, None if sc is None else dev(sc))
    ridx, rw = O.route_topk_softmax(logits, k, sc)
    np.testing.assert_array_equal(host(idx), ridx)
    np.testing.assert_array_equal(host(w), rw)
    reo, rroutes = O.build_schedule(ridx, rw, E)
    np.testing.assert_array_equal(host(eo), reo)
    r = host(routes)
    np.testing.assert_array_equal(r[:, 0], rroutes["token"])
    np.testing.assert_array_equal(r[:, 1].view(np.float32), rroutes["weight"])
    i2, w2 = gpu.route_topk(dev(logits), k, None if sc is None else dev(sc))
    eo2, routes2 = gpu.build_schedule(i2, w2, E)
    np.testing.assert_array_equal(host(eo2), host(eo))
    np.testing.assert_array_equal(host(routes2), r)


@pytest.mark.parametrize("T,E,k,H,B,pes", [(1, 128, 8, 2816, 128, True), (7, 128, 8, 2816, 128, False),
                                           (16, 128, 8, 2816, 128, True), (32, 128, 8, 2816, 128, True),
                                           (33, 128, 8, 2816, 128, False), (128, 128, 8, 2816, 128, True),
                                           (129, 128, 8, 2816, 128, False), (20, 60, 2, 512, 64, False),
                                           (9, 256, 16, 4096, 256, True), (40, 64, 4, 1024, 512, False),
                                           (3, 200, 3, 2304, 256, True), (257, 64, 4, 4096, 128, False),
                                           (600, 200, 2, 1024, 128, True), (301, 128, 8, 2816, 256, True),
                                           (2048, 128, 8, 2816, 128, True)])
def test_moe_prep(gpu, O, T, E, k, H, B, pes):
    """route top-k + softmax, the CSR schedule and the norm-quant of the MoE
    input in one call against the oracle, bit-exact: one launch up to 1024
    slots (up to 16 tokens one workgroup takes the whole top-k and schedule,
    above that the last of the top-k workgroups builds the schedule); above,
    with FWHT block 128, the top-k and the norm-quant in one
    launch and the schedule in a second (T = 129, 257, 600, 2048), else the
    separate launches (T = 301 at block 256).  Three calls in a row (the
    small launch's completion counter is reset by the workgroup that builds
    the schedule)"""
    logits = O.synth_normal_f32(70 + T, 1.0, (T, E))
    sc = O.f32_to_bf16(O.synth_normal_f32(71, 0.2, (E,)) + 1.0) if pes else None
    x = O.synth_normal_bf16(72 + T, 1.0, (T, H))
    g = O.f32_to_bf16(O.synth_normal_f32(73, 0.3, (H,)) + 1.0)
    ridx, rw = O.route_topk_softmax(logits, k, sc)
    reo, rroutes = O.build_schedule(ridx, rw, E)
    rq, rsa = O.norm_quant(x, g, B)
    for _ in range(3):
        idx, w, eo, routes, xq, sa = gpu.moe_prep(dev(logits), dev(x), dev(g), k,
                                                  None if sc is None else dev(sc), block=B)
        np.testing.assert_array_equal(host(idx), ridx)
        np.testing.assert_array_equal(host(w), rw)
        np.testing.assert_array_equal(host(eo), reo)
        r = host(routes)
        np.testing.assert_array_equal(r[:, 0], rroutes["token"])
        np.testing.assert_array_equal(r[:, 1].view(np.float32), rroutes["weight"])
        np.testing.assert_array_equal(host(xq), rq)
        np.testing.assert_array_equal(host(sa), rsa)


def test_moe_prep_two_streams(gpu, O):
    """The spread form's completion counter is per stream: two streams run
    preps of different batches at the same time, each bit-exact."""
    import torch
    E, k, H, B = 128, 8, 2816, 128
    cases = []
    for T in (32, 48):
        logits = O.synth_normal_f32(90 + T, 1.0, (T, E))
        x = O.synth_normal_bf16(91 + T, 1.0, (T, H))
        g = O.f32_to_bf16(O.synth_normal_f32(92, 0.3, (H,)) + 1.0)
        ridx, rw = O.route_topk_softmax(logits, k, None)
        reo, rroutes = O.build_schedule(ridx, rw, E)
        cases.append((dev(logits), dev(x), dev(g), ridx, rw, reo, rroutes))
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]
    for _ in range(20):
        outs = []
        for (lg, x, g, *_), st in zip(cases, streams):
            with torch.cuda.stream(st):
                outs.append(gpu.moe_prep(lg, x, g, k, None, block=B))
        torch.cuda.synchronize()
        for (_, _, _, ridx, rw, reo, rroutes), (idx, w, eo, routes, xq, sa) in zip(cases, outs):
            np.testing.assert_array_equal(host(idx), ridx)
            np.testing.assert_array_equal(host(w), rw)
            np.testing.assert_array_equal(host(eo), reo)
            r = host(routes)
            np.testing.assert_array_equal(r[:, 0], rroutes["token"])
            np.testing.assert_array_equal(r[:, 1].view(np.float32), rroutes["weight"])


def test_moe_prep_batches_in_a_row(gpu, O):
    """calls of different batch sizes after each other (grids of different
    workgroup counts share the completion counter) match the separate calls"""
    E, k, H = 128, 8, 2816
    g = O.f32_to_bf16(O.synth_normal_f32(75, 0.3, (H,)) + 1.0)
    for T in (32, 5, 64, 1, 16, 17, 32):
        logits = dev(O.synth_normal_f32(76 + T, 1.0, (T, E)))
        x = dev(O.synth_normal_bf16(77 + T, 1.0, (T, H)))
        idx, w, eo, routes, xq, sa = gpu.moe_prep(logits, x, dev(g), k)
        i2, w2, eo2, r2 = gpu.route_schedule(logits, k)
        xq2, sa2 = gpu.norm_quant(x, dev(g), 128)
        for a, b in ((idx, i2), (w, w2), (eo, eo2), (routes, r2), (xq, xq2), (sa, sa2)):
            np.testing.assert_array_equal(host(a), host(b))


@pytest.mark.parametrize("T,E,k,H,B", [(1, 128, 8, 2816, 128), (7, 128, 8, 2816, 128),
                                       (16, 128, 8, 2816, 128), (17, 128, 8, 2816, 128),
                                       (32, 128, 8, 2816, 128), (9, 256, 16, 4096, 256),
                                       (129, 128, 8, 2816, 128), (301, 128, 8, 2816, 256)])
def test_ffn_prep(gpu, O, T, E, k, H, B):
    """bq_ffn_prep = bq_moe_prep plus the dense MLP's norm-quant of the same
    rows with a second gain, against the oracle, bit-exact: the dense rows in
    more workgroups of the one prep launch (T <= 128 at top-8), or a launch of
    their own before the two-launch and separate paths (T = 129, 301).  Three
    calls in a row."""
    logits = O.synth_normal_f32(80 + T, 1.0, (T, E))
    x = O.synth_normal_bf16(81 + T, 1.0, (T, H))
    g = O.f32_to_bf16(O.synth_normal_f32(82, 0.3, (H,)) + 1.0)
    gd = O.f32_to_bf16(O.synth_normal_f32(83, 0.3, (H,)) + 1.0)
    ridx, rw = O.route_topk_softmax(logits, k, None)
    reo, rroutes = O.build_schedule(ridx, rw, E)
    rq, rsa = O.norm_quant(x, g, B)
    rdq, rdsa = O.norm_quant(x, gd, B)
    for _ in range(3):
        idx, w, eo, routes, xq, sa, dq, dsa = gpu.ffn_prep(dev(logits), dev(x), dev(g), dev(gd), k,
                                                           block=B)
        np.testing.assert_array_equal(host(idx), ridx)
        np.testing.assert_array_equal(host(w), rw)
        np.testing.assert_array_equal(host(eo), reo)
        r = host(routes)
        np.testing.assert_array_equal(r[:, 0], rroutes["token"])
        np.testing.assert_array_equal(r[:, 1].view(np.float32), rroutes["weight"])
        np.testing.assert_array_equal(host(xq), rq)
        np.testing.assert_array_equal(host(sa), rsa)
        np.testing.assert_array_equal(host(dq), rdq)
        np.testing.assert_array_equal(host(dsa), rdsa)


def test_ffn_prep_matches_separate_calls(gpu, O):
    """batches of different sizes in a row (the spread form's counter is
    shared): bq_ffn_prep = bq_moe_prep + bq_norm_quant with the dense gain"""
    E, k, H = 128, 8, 2816
    g = dev(O.f32_to_bf16(O.synth_normal_f32(85, 0.3, (H,)) + 1.0))
    gd = dev(O.f32_to_bf16(O.synth_normal_f32(86, 0.3, (H,)) + 1.0))
    for T in (32, 5, 64, 1, 16, 17, 32):
        logits = dev(O.synth_normal_f32(87 + T, 1.0, (T, E)))
        x = dev(O.synth_normal_bf16(88 + T, 1.0, (T, H)))
        outs = gpu.ffn_prep(logits, x, g, gd, k)
        ref = gpu.moe_prep(logits, x, g, k) + gpu.norm_quant(x, gd, 128)
        for a, b in zip(outs, ref):
            np.testing.assert_array_equal(host(a), host(b))


def test_build_schedule_expert_range(gpu, O):
    # expert-parallel slice [32, 64) as a rank of degree 4 would build it
    idx, w = route_table(O, 40)
    eo, routes = gpu.build_schedule(dev(idx), dev(w), 32, expert_base=32)
    sel = (idx >= 32) & (idx < 64)
    reo, rroutes = O.build_schedule(np.where(sel, idx - 32, -1).astype(np.int32), w, 32)
    np.testing.assert_array_equal(host(eo), reo)
    np.testing.assert_array_equal(host(routes)[: reo[-1], 0], rroutes["token"])


def gpu_moe(gpu, xq, xsa, idx, w, Wgu, Wd, E, H, I):
    import torch
    T, k = idx.shape
    eo, routes = gpu.build_schedule(dev(idx), dev(w), E)
    bucket = gpu.moe_phase1(xq, xsa, eo, routes, Wgu, E, T, k, I)
    bi8, bsa = gpu.block_quant(bucket, 64, True)
    accum, out = gpu.moe_phase2(bi8, bsa, eo, routes, Wd, E, T, k, H)
    torch.cuda.synchronize()
    return eo, routes, bucket, bi8, bsa, accum, out


def test_moe_golden(gpu, G):
    E, H, I = 4, 128, 64
    idx, w = G["moe_idx"], G["moe_w"]
    Wgu = gpu.ButterquantWeight(gpu.retile(dev(G["moe_gq"].reshape(-1)), E * 2 * I, H),
                                dev(G["moe_gs"]), E * 2 * I, H)
    Wd = gpu.ButterquantWeight(gpu.retile(dev(G["moe_dq"].reshape(-1)), E * H, I),
                               dev(G["moe_ds"]), E * H, I)
    eo, routes, bucket, bi8, bsa, accum, out = gpu_moe(
        gpu, dev(G["moe_xq"]), dev(G["moe_xsa"]), idx, w, Wgu, Wd, E, H, I)
    np.testing.assert_array_equal(host(eo), G["moe_eo"])
    np.testing.assert_array_equal(host(bucket), G["moe_bucket"])
    np.testing.assert_array_equal(host(bi8), G["moe_bucket_i8"])
    np.testing.assert_array_equal(host(bsa), G["moe_bucket_sa"])
    np.testing.assert_array_equal(host(accum), G["moe_accum"])
    np.testing.assert_array_equal(host(out), G["moe_out"])


@pytest.mark.parametrize("T,E,k,H,I", [(1, 4, 2, 1024, 128), (5, 8, 2, 768, 128),
                                       (40, 8, 2, 1024, 192), (300, 4, 2, 1024, 128),
                                       (600, 4, 2, 1024, 64), (129, 16, 4, 2816, 128),
                                       (64, 8, 8, 2112, 128), (20, 4, 2, 512, 64)])
def test_moe_phase1_quant(gpu, O, T, E, k, H, I):
    """bq_moe_phase1_gate_up_quant = phase 1 then the FWHT64 block-quant of
    its bucket (bit for bit), with and without the bf16 bucket: the skinny
    16-record kernel (few routes per expert) and the LDS-tiled kernel (T =
    300 / 600 over 4 experts: 150 / 300 records per expert, one and two
    m-tiles), hidden a multiple of 128 or only of 64."""
    import torch
    idx, w = O.route_topk_softmax(O.synth_normal_f32(T + 3, 1.0, (T, E)), k)
    gq, gs, Wgu = weight(gpu, O, E * 2 * I, H, 128 if H % 128 == 0 else 64, seed=9)
    gp, gcs = O.pack_and_colsum(gq)
    x = O.synth_normal_bf16(T, 1.0, (T, H))
    xq, xsa = O.norm_quant(x, np.full(H, ONE, np.uint16), 128 if H % 128 == 0 else 64)
    eo, routes = gpu.build_schedule(dev(idx), dev(w), E)
    reo, rroutes = O.build_schedule(idx, w, E)
    rb = O.moe_phase1(xq, xsa, reo, rroutes, gp, gs, gcs, I)
    rq, rsa = O.block_quant(rb, 64, True)
    n = int(reo[-1])
    bi8, bsa, bb = gpu.moe_phase1_quant(dev(xq), dev(xsa), eo, routes, Wgu, E, T, k, I, bucket=True)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(host(bb)[:n], rb)
    np.testing.assert_array_equal(host(bi8)[:n], rq)
    np.testing.assert_array_equal(host(bsa)[:n], rsa)
    bi8, bsa = gpu.moe_phase1_quant(dev(xq), dev(xsa), eo, routes, Wgu, E, T, k, I)
    np.testing.assert_array_equal(host(bi8)[:n], rq)
    np.testing.assert_array_equal(host(bsa)[:n], rsa)


# (T, E, top_k, hidden, expert inter, dense inter): the experts in the 16-row
# kernels (T <= 40 here; 1..10 routes per expert) or the LDS-tiled ones (T =
# 300 and 129 over 4 experts, the dense gate/up then in 64-token workgroups,
# the last one partial); dense_inter narrower than, a multiple of, and not a
# multiple of the experts' 64-column groups; ragged 16-token tiles
FFN_CASES = [(1, 8, 2, 1024, 128, 192), (16, 8, 2, 1024, 128, 320), (17, 16, 4, 2816, 128, 256),
             (40, 8, 2, 1024, 192, 128), (300, 4, 2, 1024, 128, 192), (129, 4, 2, 1024, 128, 320)]


def _dense_gate_up_ref(O, dq, dsa, qg, sg, qu, su, DI):
    """oracle chain of the dense MLP up to the down projection's activation:
    gate and up linears (bf16), gelu_gate_up, FWHT64 block-quant"""
    pg, cg = O.pack_and_colsum(qg)
    pu, cu = O.pack_and_colsum(qu)
    rg, _ = O.linear(dq, dsa, pg, sg, cg, DI)
    ru, _ = O.linear(dq, dsa, pu, su, cu, DI)
    return O.block_quant(O.gelu_gate_up(rg, ru), 64, True)


@pytest.mark.parametrize("T,E,k,H,I,DI", FFN_CASES)
def test_ffn_gate_up(gpu, O, T, E, k, H, I, DI):
    """bq_ffn_gate_up = bq_moe_phase1_gate_up_quant (bit for bit) plus the
    dense MLP's gate and up linears, GELU-tanh product and FWHT64 block-quant
    against the oracle, bit-exact; two calls in a row."""
    import torch
    idx, w = O.route_topk_softmax(O.synth_normal_f32(T + 5, 1.0, (T, E)), k)
    _, _, Wgu = weight(gpu, O, E * 2 * I, H, 128, seed=9)
    ones = np.full(H, ONE, np.uint16)
    xq, xsa = O.norm_quant(O.synth_normal_bf16(T + 1, 1.0, (T, H)), ones, 128)
    dq, dsa = O.norm_quant(O.synth_normal_bf16(T + 2, 1.0, (T, H)), ones, 128)
    (qg, sg, Wg), (qu, su, Wu) = (weight(gpu, O, DI, H, 128, seed=sd) for sd in (21, 22))
    rdq, rdsa = _dense_gate_up_ref(O, dq, dsa, qg, sg, qu, su, DI)
    eo, routes = gpu.build_schedule(dev(idx), dev(w), E)
    mi8, msa = gpu.moe_phase1_quant(dev(xq), dev(xsa), eo, routes, Wgu, E, T, k, I)
    n = int(host(eo)[-1])
    for _ in range(2):
        bi8, bsa, di8, dsa_ = gpu.ffn_gate_up(dev(xq), dev(xsa), eo, routes, Wgu, E, T, k, I,
                                              dev(dq), dev(dsa), Wg, Wu)
        torch.cuda.synchronize()
        np.testing.assert_array_equal(host(bi8)[:n], host(mi8)[:n])
        np.testing.assert_array_equal(host(bsa)[:n], host(msa)[:n])
        np.testing.assert_array_equal(host(di8), rdq)
        np.testing.assert_array_equal(host(dsa_), rdsa)


@pytest.mark.parametrize("T,E,k,H,I,DI", FFN_CASES)
def test_ffn_down(gpu, O, T, E, k, H, I, DI):
    """bq_ffn_down = bq_moe_phase2_down (bit for bit) plus the dense MLP's
    per-block (B = 64) down projection against the oracle's block linear,
    bit-exact; two calls in a row."""
    import torch
    idx, w = O.route_topk_softmax(O.synth_normal_f32(T + 5, 1.0, (T, E)), k)
    _, _, Wd = weight(gpu, O, E * H, I, 64, seed=11)
    bi8, bsa = O.block_quant(O.synth_normal_bf16(T + 7, 1.0, (T * k, I)), 64, True)
    di8, dsa = O.block_quant(O.synth_normal_bf16(T + 8, 1.0, (T, DI)), 64, True)
    qd, sd, Wdd = weight(gpu, O, H, DI, 64, seed=23)
    pd, cd = O.pack_and_colsum(qd, 64, False)
    rdo, _ = O.block_linear(di8, dsa, pd, sd, cd, H, 64)
    eo, routes = gpu.build_schedule(dev(idx), dev(w), E)
    macc, mout = gpu.moe_phase2(dev(bi8), dev(bsa), eo, routes, Wd, E, T, k, H)
    for _ in range(2):
        acc, out, do = gpu.ffn_down(dev(bi8), dev(bsa), eo, routes, Wd, E, T, k, H, dev(di8),
                                    dev(dsa), Wdd)
        torch.cuda.synchronize()
        np.testing.assert_array_equal(host(acc), host(macc))
        np.testing.assert_array_equal(host(out), host(mout))
        np.testing.assert_array_equal(host(do), rdo)


def test_ffn_model_shape_decode(gpu, O, moe_model):
    """The batch-16 decoder layer's FFN at the model's shapes (128 experts,
    top-8, hidden 2816, expert inter 704, dense inter 2112): bq_ffn_gate_up and
    bq_ffn_down against the separate MoE calls and the oracle's dense chain
    (gate, up, gelu_gate_up, FWHT64 block-quant, per-block down)."""
    import torch
    m = moe_model
    E, H, I, T, k, DI = m["E"], m["H"], m["I"], 16, 8, 2112
    ones = np.full(H, ONE, np.uint16)
    idx, w = route_table(O, T)
    xq, xsa = O.norm_quant(O.synth_normal_bf16(31, 1.0, (T, H)), ones, 128)
    dq, dsa = O.norm_quant(O.synth_normal_bf16(32, 1.0, (T, H)), ones, 128)
    (qg, sg, Wg), (qu, su, Wu) = (weight(gpu, O, DI, H, 128, seed=sd) for sd in (24, 25))
    qd, sd, Wdd = weight(gpu, O, H, DI, 64, seed=26)
    rdq, rdsa = _dense_gate_up_ref(O, dq, dsa, qg, sg, qu, su, DI)
    pd, cd = O.pack_and_colsum(qd, 64, False)
    rdo, _ = O.block_linear(rdq, rdsa, pd, sd, cd, H, 64)
    eo, routes = gpu.build_schedule(dev(idx), dev(w), E)
    mi8, msa = gpu.moe_phase1_quant(dev(xq), dev(xsa), eo, routes, m["Wgu"], E, T, k, I)
    macc, mout = gpu.moe_phase2(mi8, msa, eo, routes, m["Wd"], E, T, k, H)
    bi8, bsa, di8, dsa_ = gpu.ffn_gate_up(dev(xq), dev(xsa), eo, routes, m["Wgu"], E, T, k, I,
                                          dev(dq), dev(dsa), Wg, Wu)
    acc, out, do = gpu.ffn_down(bi8, bsa, eo, routes, m["Wd"], E, T, k, H, di8, dsa_, Wdd)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(host(bi8), host(mi8))
    np.testing.assert_array_equal(host(bsa), host(msa))
    np.testing.assert_array_equal(host(di8), rdq)
    np.testing.assert_array_equal(host(dsa_), rdsa)
    np.testing.assert_array_equal(host(acc), host(macc))
    np.testing.assert_array_equal(host(out), host(mout))
    np.testing.assert_array_equal(host(do), rdo)


def test_moe_duplicate_experts(gpu, O):
    """A token that lists an expert more than once (the router pads a token
    with fewer than top_k valid logits with expert 0, moe_router.mojo:266):
    the schedule keeps its records in k order and phase 2 adds both, in
    record order, as the reference's route loop does (moe.mojo:259-282)."""
    E, H, I, T, k = 8, 256, 128, 6, 4
    rng = np.random.default_rng(5)
    idx = np.stack([rng.permutation(E)[:k] for _ in range(T)]).astype(np.int32)
    idx[0] = [3, 3, 0, 0]
    idx[2] = [0, 5, 0, 0]
    idx[5, 1] = idx[5, 0]
    w = rng.random((T, k)).astype(np.float32)
    gq, gs, Wgu = weight(gpu, O, E * 2 * I, H, 128, seed=7)
    dq, ds, Wd = weight(gpu, O, E * H, I, 64, seed=8)
    gp, gcs = O.pack_and_colsum(gq)
    dp, dcs = O.pack_and_colsum(dq, 64, False)
    x = O.synth_normal_bf16(1, 1.0, (T, H))
    xq, xsa = O.norm_quant(x, np.full(H, ONE, np.uint16), 128)
    eo, routes, bucket, bi8, bsa, accum, out = gpu_moe(gpu, dev(xq), dev(xsa), idx, w, Wgu, Wd,
                                                       E, H, I)
    reo, rroutes = O.build_schedule(idx, w, E)
    np.testing.assert_array_equal(host(eo), reo)
    np.testing.assert_array_equal(host(routes)[:, 0], rroutes["token"])
    rb = O.moe_phase1(xq, xsa, reo, rroutes, gp, gs, gcs, I)
    np.testing.assert_array_equal(host(bucket), rb)
    rbq, rbsa = O.block_quant(rb, 64, True)
    racc, rout = O.moe_phase2(rbq, rbsa, reo, rroutes, T, dp, ds, dcs, H)
    np.testing.assert_array_equal(host(accum), racc)
    np.testing.assert_array_equal(host(out), rout)


@pytest.mark.parametrize("T,H", [(5, 832), (3, 320), (300, 832)])
def test_moe_combine_ragged_hidden(gpu, O, T, H):
    """Phase 2 with hidden not a multiple of the combine's 256-column
    chunks (a partial last chunk below 256 tokens, whole rows above)
    against the oracle, bit-exact."""
    E, I, k = 8, 128, 2
    idx, w = O.route_topk_softmax(O.synth_normal_f32(T + 11, 1.0, (T, E)), k)
    B = 128 if H % 128 == 0 else 64
    gq, gs, Wgu = weight(gpu, O, E * 2 * I, H, B, seed=21)
    dq, ds, Wd = weight(gpu, O, E * H, I, 64, seed=22)
    gp, gcs = O.pack_and_colsum(gq)
    dp, dcs = O.pack_and_colsum(dq, 64, False)
    x = O.synth_normal_bf16(T + 12, 1.0, (T, H))
    xq, xsa = O.norm_quant(x, np.full(H, ONE, np.uint16), B)
    eo, routes, bucket, bi8, bsa, accum, out = gpu_moe(gpu, dev(xq), dev(xsa), idx, w, Wgu, Wd,
                                                       E, H, I)
    reo, rroutes = O.build_schedule(idx, w, E)
    rb = O.moe_phase1(xq, xsa, reo, rroutes, gp, gs, gcs, I)
    np.testing.assert_array_equal(host(bucket), rb)
    rbq, rbsa = O.block_quant(rb, 64, True)
    racc, rout = O.moe_phase2(rbq, rbsa, reo, rroutes, T, dp, ds, dcs, H)
    np.testing.assert_array_equal(host(accum), racc)
    np.testing.assert_array_equal(host(out), rout)


def test_moe_model_shape_decode(gpu, O, moe_model):
    """Gemma-4-26B-A4B expert shapes (H=2816, I=704, 128 experts, top-8), T=8."""
    m = moe_model
    E, H, I, T = m["E"], m["H"], m["I"], 8
    x = O.synth_normal_bf16(1, 1.0, (T, H))
    idx, w = route_table(O, T)
    xq, xsa = gpu.norm_quant(dev(x), dev(np.full(H, ONE, np.uint16)), 128)
    eo, routes, bucket, bi8, bsa, accum, out = gpu_moe(gpu, xq, xsa, idx, w, m["Wgu"], m["Wd"], E, H, I)
    reo, rroutes = O.build_schedule(idx, w, E)
    rb = O.moe_phase1(host(xq), host(xsa), reo, rroutes, m["gp"], m["gs"], m["gcs"], I)
    np.testing.assert_array_equal(host(bucket), rb)
    rbq, rbsa = O.block_quant(rb, 64, True)
    np.testing.assert_array_equal(host(bi8), rbq)
    np.testing.assert_array_equal(host(bsa), rbsa)
    racc, rout = O.moe_phase2(rbq, rbsa, reo, rroutes, T, m["dp"], m["ds"], m["dcs"], H)
    np.testing.assert_array_equal(host(accum), racc)
    np.testing.assert_array_equal(host(out), rout)
    tol_check(host(accum), racc)
