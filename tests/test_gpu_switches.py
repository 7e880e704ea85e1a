"""GPU parity of the library's non-default tuning paths (BQ_* switches read at
bq_init), each against the CPU oracle, bit-exact: every switch value the
library still accepts selects a code path that stays correct.  The default
paths are covered by the other GPU tests."""
import numpy as np
import pytest

from test_gpu_parity import dev, host, weight

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

