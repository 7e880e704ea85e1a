"""GPU parity of the butterquant vocabulary head and embedding (libbq.so
through its C ABI) against the CPU oracle: head prep (per-block norm-quant,
butterquant_kernels/head.mojo:25-78), flash sample (head.mojo:81-167 +
kernels/flash_sample.mojo:221-265) and the embedding lookup
(butterquant_kernels/embedding.mojo:21-96).

Bar: bit-exact for codes, scales, bf16 embeddings, sampled tokens, top-n
values and indices and n.  logz (a log-sum-exp whose f32 rounding follows
how the vocabulary is partitioned -- the reference's worker split and the
GPU's workgroup split differ, and a sequential f32 sum over 262144 terms
drifts by ~1e-5) within 2e-5 relative, inside the 1e-3 bar for f32 outputs.
"""
import numpy as np
import pytest

from test_gpu_parity import dev, host

pytestmark = pytest.mark.gpu


def upload_head(gpu, w, ws):
    V, H = w.shape
    t = gpu.retile(dev(w.reshape(-1)), V, H)
    return gpu.ButterquantWeight(t, dev(ws), V, H)


def run_sample(gpu, O, xq, xsa, W, params, block=128, vocab_base=0):
    import torch
    pr = torch.from_numpy(np.ascontiguousarray(params).view(np.uint8).reshape(len(params), -1)).cuda()
    out = gpu.flash_sample(dev(xq), dev(xsa), W, W.scale, pr, block=block, vocab_base=vocab_base)
    return host(out).view(O.OUTCOME_DT).reshape(-1)


def check_outcomes(got, ref):
    np.testing.assert_array_equal(got["token_id"], ref["token_id"])
    np.testing.assert_array_equal(got["n"], ref["n"])
    np.testing.assert_array_equal(got["topn_idx"], ref["topn_idx"])
    np.testing.assert_array_equal(got["topn_val"].view(np.uint32), ref["topn_val"].view(np.uint32))
    np.testing.assert_allclose(got["logz"], ref["logz"], rtol=2e-5)


@pytest.mark.parametrize("R,H,B", [(1, 2816, 128), (5, 2816, 128), (32, 2816, 128),
                                   (2, 4096, 128), (4, 256, 128), (3, 1280, 128),
                                   (2, 640, 128), (3, 512, 64), (3, 512, 256), (2, 1024, 512)])
def test_head_prep(gpu, O, R, H, B):
    """FWHT block 128 with hidden % 256 == 0 takes the 8-values-per-lane form
    (a block's scale is a max over 16 lanes); 640 and the other blocks take
    the wave-per-block form. The last row's second block is all zeros: its
    scale and codes are 0."""
    x = O.synth_normal_bf16(40 + R, 1.0, (R, H))
    x[-1, B:2 * B] = 0
    g = O.f32_to_bf16(np.linspace(0.5, 1.5, H).astype(np.float32))
    q, sa = gpu.head_prep(dev(x), dev(g), B)
    rq, rsa = O.norm_quant(x, g, B, per_block=True)
    np.testing.assert_array_equal(host(q), rq)
    np.testing.assert_array_equal(host(sa), rsa)


def head_inputs(O, R, V, H, seed, block=128, coarse=False):
    rng = np.random.default_rng(seed)
    x = O.f32_to_bf16(rng.standard_normal((R, H)).astype(np.float32))
    xq, xsa = O.norm_quant(x, np.full(H, 0x3F80, np.uint16), block, per_block=True)
    if coarse:
        # few distinct logits: long runs of exact ties in the top-n
        w = (rng.integers(-1, 2, (V, H)) * 3).astype(np.int8)
        ws = np.full((V, H // block), 1e-4, np.float32)
    else:
        w = rng.integers(-127, 128, (V, H), dtype=np.int8)
        ws = (rng.random((V, H // block)) / 127 / 30).astype(np.float32)
    return xq, xsa, w, ws


@pytest.mark.parametrize("R,V,H,coarse", [(1, 4096, 2816, False), (4, 8192, 2816, False),
                                          (17, 2048, 512, False), (3, 4096, 512, True),
                                          (2, 160, 256, False)])
def test_flash_sample(gpu, O, R, V, H, coarse):
    xq, xsa, w, ws = head_inputs(O, R, V, H, 50 + R, coarse=coarse)
    rng = np.random.default_rng(R)
    params = O.sampling_params(
        R, temperature=rng.choice([1.0, 0.7, 1.5], R), min_p=rng.choice([0.0, 0.0, 0.05], R),
        top_k=rng.choice([0, 0, 40, 1], R), seed=rng.integers(0, 2 ** 62, R),
        n_keep=rng.choice([256, 20, 0], R), greedy=rng.random(R) < 0.3)
    W = upload_head(gpu, w, ws)
    got = run_sample(gpu, O, xq, xsa, W, params)
    check_outcomes(got, O.flash_sample(xq, xsa, w, ws, params))


def test_flash_sample_full_vocab(gpu, O):
    # the model's head: 262144 x 2816, per-block B = 128, two rows, one greedy
    R, V, H = 2, 262144, 2816
    xq, xsa, w, ws = head_inputs(O, R, V, H, 77)
    params = O.sampling_params(R, seed=[123, 456], greedy=[False, True], top_k=[40, 0],
                               min_p=[0.05, 0.0])
    W = upload_head(gpu, w, ws)
    got = run_sample(gpu, O, xq, xsa, W, params)
    check_outcomes(got, O.flash_sample(xq, xsa, w, ws, params))


def test_flash_sample_vocab_shard(gpu, O):
    # rank 1 of a vocabulary split: indices and noise counters are global
    R, V, H = 2, 1024, 512
    xq, xsa, w, ws = head_inputs(O, R, V, H, 81)
    params = O.sampling_params(R, seed=[5, 6])
    W = upload_head(gpu, w, ws)
    got = run_sample(gpu, O, xq, xsa, W, params, vocab_base=4096)
    check_outcomes(got, O.flash_sample(xq, xsa, w, ws, params, vocab_base=4096))
    assert (got["token_id"] >= 4096).all()


@pytest.mark.parametrize("H,B", [(2816, 128), (512, 64), (1024, 256), (1024, 512)])
def test_embed_lookup(gpu, O, H, B):
    rng = np.random.default_rng(H + B)
    rows = 96
    w = rng.integers(-127, 128, (rows, H), dtype=np.int8)
    ws = (rng.random((rows, H // B)) * 0.01).astype(np.float32)
    tok = np.array([0, 5, 95, 5, 17, 94], np.int32)
    W = upload_head(gpu, w, ws)
    scale = O.embed_scale(2816)
    got = gpu.embed_lookup(dev(tok), W, W.scale, B, scale=scale)
    np.testing.assert_array_equal(host(got), O.embed_lookup(tok, w, ws, B, scale=scale))
    # shard 1 of two (rows [48, 96)): tokens below 48 or above 95 give zero rows
    W1 = upload_head(gpu, np.ascontiguousarray(w[48:]), np.ascontiguousarray(ws[48:]))
    got1 = gpu.embed_lookup(dev(tok), W1, W1.scale, B, scale=scale, shard_rows=48, rank=1)
    np.testing.assert_array_equal(host(got1), O.embed_lookup(tok, w[48:], ws[48:], B, scale=scale,
                                                             shard_rows=48, rank=1))
    # negative (padding) ids and ids past every shard: zero rows at rank 0 and 1
    odd = np.array([-1, -48, -49, -(2 ** 31), 96, 10 ** 6, 3], np.int32)
    for rank, Wr in ((0, upload_head(gpu, np.ascontiguousarray(w[:48]), np.ascontiguousarray(ws[:48]))),
                     (1, W1)):
        g = host(gpu.embed_lookup(dev(odd), Wr, Wr.scale, B, scale=scale, shard_rows=48, rank=rank))
        np.testing.assert_array_equal(g, O.embed_lookup(odd, w[48 * rank:48 * rank + 48],
                                                        ws[48 * rank:48 * rank + 48], B,
                                                        scale=scale, shard_rows=48, rank=rank))
        assert (g[:6] == 0).all()
