"""GPU parity at the benchmark configurations' own shapes (Gemma-4-26B-A4B,
modeling/gemma4_common.mojo): every output element compared bit for bit.

  * the quantized projections of one decoder layer at decode batch 16:
    sliding q/k/v 4096/2048/2048 through bq_qkv and o_proj 2816 x 4096
    (per-block 256, no runtime FWHT); full q 8192 / k 1024 and o_proj
    2816 x 8192 (per-block 512); the dense MLP's gate/up 2112 and down
    2816 x 2112 (per-block 64) -- butterquant_kernels/linear.mojo:119-326,
    modeling/gemma_4_moe_bq.mojo:515-522, 618-620;
  * the 128-expert top-8 MoE layer (butterquant_kernels/moe.mojo:25-335) at
    16 and 32 tokens against the oracle, and at 2048 tokens -- every bucket
    row, every accum and out element -- against the VNNI port of the
    reference CPU path (oracle/cpu_baseline.c), which
    tests/test_cpu_baseline.py pins bit for bit to the oracle.
"""
import os

import numpy as np
import pytest

from test_gpu_parity import dev, host, route_table, gpu_moe, tol_check

pytestmark = pytest.mark.gpu
ONE = 0x3F80
H = 2816
NCPU = max(1, min(16, len(os.sched_getaffinity(0))))


def quantized(gpu, O, n, k, block, seed):
    wf = O.bf16_to_f32(O.synth_normal_bf16(seed, 0.02, (n, k)))
    q, s = O.rotate_and_quant(wf, block)
    return q, s, gpu.ButterquantWeight(gpu.retile(dev(q.reshape(-1)), n, k), dev(s), n, k)


@pytest.fixture(scope="module")
def batch16(O):
    x = O.synth_normal_bf16(1, 1.0, (16, H))
    return O.norm_quant(x, np.full(H, ONE, np.uint16), 128)


@pytest.mark.parametrize("qn,kvn", [(4096, 2048)])
def test_qkv_sliding_b16(gpu, O, batch16, qn, kvn):
    xq, sa = batch16
    ws = [quantized(gpu, O, n, H, 128, seed) for n, seed in ((qn, 40), (kvn, 41), (kvn, 42))]
    outs = gpu.qkv(dev(xq), dev(sa), *(w[2] for w in ws))
    for o, (q, s, _) in zip(outs, ws):
        p, cs = O.pack_and_colsum(q)
        rb, _ = O.linear(xq, sa, p, s, cs, q.shape[0])
        np.testing.assert_array_equal(host(o), rb)


@pytest.mark.parametrize("n,seed", [(8192, 43), (1024, 44), (2112, 45)])
def test_linear_b16(gpu, O, batch16, n, seed):
    """full-attention q (8192) and k (1024), dense gate/up (2112)"""
    xq, sa = batch16
    q, s, W = quantized(gpu, O, n, H, 128, seed)
    ob, of = gpu.linear(dev(xq), dev(sa), W, want_f32=True)
    p, cs = O.pack_and_colsum(q)
    rb, rf = O.linear(xq, sa, p, s, cs, n)
    np.testing.assert_array_equal(host(of), rf)
    np.testing.assert_array_equal(host(ob), rb)
    tol_check(host(of), rf)


@pytest.mark.parametrize("K,B,fwht", [(4096, 256, False), (8192, 512, False), (2112, 64, True)])
def test_block_linear_b16(gpu, O, K, B, fwht):
    """o_proj 2816 x 4096 (B = 256) and 2816 x 8192 (B = 512), activations
    block-quantized without FWHT; dense down 2816 x 2112 (B = 64, FWHT)"""
    q, s, W = quantized(gpu, O, H, K, B, 46 + B)
    x = O.synth_normal_bf16(47, 1.0, (16, K))
    xq, sa = gpu.block_quant(dev(x), B, fwht)
    rq, rsa = O.block_quant(x, B, fwht)
    np.testing.assert_array_equal(host(xq), rq)
    np.testing.assert_array_equal(host(sa), rsa)
    ob, of = gpu.block_linear(xq, sa, W, B, want_f32=True)
    p, cs = O.pack_and_colsum(q, B, False)
    rb, rf = O.block_linear(rq, rsa, p, s, cs, H, B)
    np.testing.assert_array_equal(host(of), rf)
    np.testing.assert_array_equal(host(ob), rb)


@pytest.mark.parametrize("T", [16, 32])
def test_moe_model_shape_batches(gpu, O, moe_model, T):
    """The 128-expert layer at decode batch 16 (config 5's MoE) and 32
    (config 3), from hidden states and router logits, every output element."""
    m = moe_model
    E, I = m["E"], m["I"]
    x = O.synth_normal_bf16(1, 1.0, (T, H))
    idx, w = route_table(O, T)
    xq, xsa = gpu.norm_quant(dev(x), dev(np.full(H, ONE, np.uint16)), 128)
    rxq, rxsa = O.norm_quant(x, np.full(H, ONE, np.uint16), 128)
    np.testing.assert_array_equal(host(xq), rxq)
    eo, routes, bucket, bi8, bsa, accum, out = gpu_moe(gpu, xq, xsa, idx, w, m["Wgu"], m["Wd"], E, H, I)
    reo, rroutes = O.build_schedule(idx, w, E)
    np.testing.assert_array_equal(host(eo), reo)
    rb = O.moe_phase1(rxq, rxsa, reo, rroutes, m["gp"], m["gs"], m["gcs"], I)
    np.testing.assert_array_equal(host(bucket), rb)
    rbq, rbsa = O.block_quant(rb, 64, True)
    np.testing.assert_array_equal(host(bi8), rbq)
    np.testing.assert_array_equal(host(bsa), rbsa)
    fi8, fsa = gpu.moe_phase1_quant(xq, xsa, eo, routes, m["Wgu"], E, T, 8, I)
    np.testing.assert_array_equal(host(fi8), rbq)
    np.testing.assert_array_equal(host(fsa), rbsa)
    racc, rout = O.moe_phase2(rbq, rbsa, reo, rroutes, T, m["dp"], m["ds"], m["dcs"], H)
    np.testing.assert_array_equal(host(accum), racc)
    np.testing.assert_array_equal(host(out), rout)
    tol_check(host(accum), racc)


def test_moe_prefill_full(gpu, O, moe_model):
    """T = 2048 (config 4): the whole layer's outputs -- all 16384 bucket
    rows, their block-quantized codes and scales, every accum and out element
    -- against the VNNI port of the reference path on the host cores."""
    m = moe_model
    E, I, T = m["E"], m["I"], 2048
    x = O.synth_normal_bf16(1, 1.0, (T, H))
    idx, w = route_table(O, T)
    print(f"moe prefill T={T}: GPU layer", flush=True)
    xq, xsa = gpu.norm_quant(dev(x), dev(np.full(H, ONE, np.uint16)), 128)
    eo, routes, bucket, bi8, bsa, accum, out = gpu_moe(gpu, xq, xsa, idx, w, m["Wgu"], m["Wd"], E, H, I)
    print(f"moe prefill T={T}: CPU port on {NCPU} threads", flush=True)
    rxq, rxsa = O.cpu_norm_quant(x, np.full(H, ONE, np.uint16), 128, NCPU)
    np.testing.assert_array_equal(host(xq), rxq)
    np.testing.assert_array_equal(host(xsa), rxsa)
    reo, rroutes = O.build_schedule(idx, w, E)
    np.testing.assert_array_equal(host(eo), reo)
    counts = np.diff(reo)
    assert counts.min() != counts.max()  # uneven histogram
    rb = O.cpu_moe_phase1(rxq, rxsa, reo, rroutes, m["gp"], m["gs"], m["gcs"], I, NCPU)
    np.testing.assert_array_equal(host(bucket), rb)
    rbq, rbsa = O.cpu_block_quant(rb, 64, True, NCPU)
    np.testing.assert_array_equal(host(bi8), rbq)
    np.testing.assert_array_equal(host(bsa), rbsa)
    # the fused phase 1 + block-quant (the benchmark's path) gives the same codes
    print(f"moe prefill T={T}: fused phase 1 + block-quant", flush=True)
    fi8, fsa = gpu.moe_phase1_quant(xq, xsa, eo, routes, m["Wgu"], E, T, 8, I)
    np.testing.assert_array_equal(host(fi8), rbq)
    np.testing.assert_array_equal(host(fsa), rbsa)
    racc, rout = O.cpu_moe_phase2(rbq, rbsa, reo, rroutes, T, m["dp"], m["ds"], m["dcs"], H, 64, NCPU)
    np.testing.assert_array_equal(host(accum), racc)
    np.testing.assert_array_equal(host(out), rout)
    tol_check(host(accum), racc)
