"""GPU parity of the MoE router (libbq.so through its C ABI) against the CPU
oracle: router logits (RouterExpertKernel, kernels/moe_router.mojo:164-187)
and top-k + softmax merge (insert_candidate :43-57, RouterMergeKernel
:248-293).

Bar: bit-exact.  Route indices compare as integers, logits and weights as
f32 bit patterns; a NaN weight (only from +inf logits, where the x86
reference produces its own NaN encoding) compares by position.
"""
import numpy as np
import pytest

from test_gpu_parity import dev, host

pytestmark = pytest.mark.gpu


def same_f32(got, ref):
    got = np.asarray(got, np.float32)
    ref = np.asarray(ref, np.float32)
    nan = np.isnan(ref)
    np.testing.assert_array_equal(np.isnan(got), nan)
    np.testing.assert_array_equal(got[~nan].view(np.uint32), ref[~nan].view(np.uint32))


def check_route(gpu, O, logits, k, scale=None):
    idx, w = gpu.route_topk(dev(logits), k, None if scale is None else dev(scale))
    ridx, rw = O.route_topk_softmax(logits, k, per_expert_scale=scale)
    np.testing.assert_array_equal(host(idx), ridx)
    same_f32(host(w), rw)


@pytest.mark.parametrize("T", [1, 32, 2048])
def test_route_topk_normal(gpu, O, T):
    # N(0,1) logits, 128 experts, top-8, per_expert_scale 1 (MoE decode and
    # prefill workloads)
    logits = O.synth_normal_f32(2, 1.0, (T, 128))
    check_route(gpu, O, logits, 8)
    check_route(gpu, O, logits, 8, np.full(128, 0x3F80, np.uint16))


@pytest.mark.parametrize("E,k", [(3, 8), (64, 1), (100, 8), (128, 16), (300, 8), (1024, 2),
                                 (1000, 16)])
def test_route_topk_shapes_ties_specials(gpu, O, E, k):
    rng = np.random.default_rng(E * 31 + k)
    T = 77
    # coarse logits force many exact ties (lower expert first)
    logits = (np.round(rng.standard_normal((T, E)) * 2) / 2).astype(np.float32)
    specials = np.array([np.nan, -np.inf, -1e30, -2e30, -1e29, 0.0, -0.0], np.float32)
    mask = rng.random((T, E)) < 0.15
    logits[mask] = rng.choice(specials, mask.sum())
    logits[0] = np.nan                      # no valid candidate: k sentinels
    logits[1, :] = -np.inf
    logits[1, E // 2] = 1.5                 # one valid candidate
    logits[2] = -0.0
    logits[2, ::3] = 0.0                    # +-0 ties
    logits[3] = 7.0                         # all equal
    scale = O.f32_to_bf16((1 + 0.3 * rng.standard_normal(E)).astype(np.float32))
    check_route(gpu, O, logits, k)
    check_route(gpu, O, logits, k, scale)


def test_route_topk_inf(gpu, O):
    # +inf winners make inf - inf in the softmax; weights may be NaN
    logits = O.synth_normal_f32(5, 1.0, (8, 128))
    logits[0, 7] = np.inf
    logits[1, [3, 9]] = np.inf
    logits[2, 5] = -np.inf
    check_route(gpu, O, logits, 8)


@pytest.mark.parametrize("T,H,E", [(1, 2816, 128), (32, 2816, 128), (300, 2816, 128),
                                   (7, 192, 37), (260, 128, 20), (3, 64, 5)])
def test_router_logits(gpu, O, T, H, E):
    rng = np.random.default_rng(T + H + E)
    x = O.f32_to_bf16(rng.standard_normal((T, H)).astype(np.float32))
    proj = O.f32_to_bf16(0.02 * rng.standard_normal((E, H)).astype(np.float32))
    rs = O.f32_to_bf16((1 + 0.1 * rng.standard_normal(H)).astype(np.float32))
    got = host(gpu.router_logits(dev(x), dev(proj), dev(rs)))
    same_f32(got, O.router_logits(x, proj, rs))


def test_router_to_schedule(gpu, O):
    # hidden -> logits -> top-8 softmax -> CSR schedule, all on the GPU
    T, H, E, k = 64, 2816, 128, 8
    rng = np.random.default_rng(11)
    x = O.f32_to_bf16(rng.standard_normal((T, H)).astype(np.float32))
    proj = O.f32_to_bf16(0.02 * rng.standard_normal((E, H)).astype(np.float32))
    rs = O.f32_to_bf16((1 + 0.1 * rng.standard_normal(H)).astype(np.float32))
    pes = O.f32_to_bf16((1 + 0.1 * rng.standard_normal(E)).astype(np.float32))
    lg = gpu.router_logits(dev(x), dev(proj), dev(rs))
    idx, w = gpu.route_topk(lg, k, dev(pes))
    eo, routes = gpu.build_schedule(idx, w, E)
    ridx, rw = O.route_topk_softmax(O.router_logits(x, proj, rs), k, per_expert_scale=pes)
    reo, rroutes = O.build_schedule(ridx, rw, E)
    np.testing.assert_array_equal(host(eo), reo)
    r = host(routes)
    np.testing.assert_array_equal(r[:, 0], rroutes["token"])
    np.testing.assert_array_equal(r[:, 1].view(np.float32).view(np.uint32),
                                  rroutes["weight"].view(np.uint32))
