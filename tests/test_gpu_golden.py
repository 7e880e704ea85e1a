"""GPU outputs of the widened rows against the committed fixtures
(tests/golden/golden.npz, written by the oracle): the MoE router, the bq
vocabulary head and embedding, and the int8-KV attention prep and attention.
Bar: bit-exact (the head's logz within 2e-5, a partition-dependent f32 sum)."""
import os

import numpy as np
import pytest

from test_gpu_parity import dev, host

pytestmark = pytest.mark.gpu
GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "golden.npz")


@pytest.fixture(scope="module")
def G():
    return dict(np.load(GOLDEN, allow_pickle=False))


def test_router_golden(gpu, G):
    import torch
    logits = gpu.router_logits(dev(G["router_x"]), dev(G["router_proj"]), dev(G["router_scale"]))
    idx, w = gpu.route_topk(logits, 2, dev(G["router_pes"]))
    torch.cuda.synchronize()
    np.testing.assert_array_equal(host(logits).view(np.uint32), G["router_logits"].view(np.uint32))
    np.testing.assert_array_equal(host(idx), G["router_idx"])
    np.testing.assert_array_equal(host(w).view(np.uint32), G["router_w"].view(np.uint32))


def test_head_and_embedding_golden(gpu, O, G):
    import torch
    V, H = G["head_w"].shape
    W = gpu.ButterquantWeight(gpu.retile(dev(G["head_w"].reshape(-1)), V, H), dev(G["head_ws"]), V, H)
    params = torch.from_numpy(G["head_params"].reshape(2, -1).copy()).cuda()
    out = host(gpu.flash_sample(dev(G["head_xq"]), dev(G["head_xsa"]), W, W.scale, params))
    got = out.view(O.OUTCOME_DT).reshape(-1)
    ref = G["head_outcome"].view(O.OUTCOME_DT).reshape(-1)
    for f in ("token_id", "n", "topn_idx"):
        np.testing.assert_array_equal(got[f], ref[f])
    np.testing.assert_array_equal(got["topn_val"].view(np.uint32), ref["topn_val"].view(np.uint32))
    np.testing.assert_allclose(got["logz"], ref["logz"], rtol=2e-5)
    emb = gpu.embed_lookup(dev(G["embed_tokens"]), W, W.scale, 128, scale=O.embed_scale(2816))
    np.testing.assert_array_equal(host(emb), G["embed_out"])


def test_attention_golden(gpu, G):
    import torch
    nq, nkv, hd, page = 4, 2, 128, 16
    kc, ks = dev(G["attn_kc_in"]), dev(G["attn_ks_in"])
    vc, vs = dev(G["attn_vc_in"]), dev(G["attn_vs_in"])
    runs, rows = dev(G["attn_runs"]), dev(G["attn_rows"])
    qi, qb, fq = gpu.attn_prep(dev(G["attn_q"]), dev(G["attn_k"]), dev(G["attn_v"]),
                               dev(G["attn_qn"]), dev(G["attn_kn"]), kc, ks, vc, vs,
                               dev(G["attn_cos"]), dev(G["attn_sin"]), runs, rows, nq, nkv, hd,
                               64, 64, 4, page - 1, -1)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(host(qi), G["attn_qi"])
    np.testing.assert_array_equal(host(qb).view(np.uint32), G["attn_qb"].view(np.uint32))
    np.testing.assert_array_equal(host(fq).view(np.uint32), G["attn_fq"].view(np.uint32))
    for name in ("kc", "vc"):
        np.testing.assert_array_equal(host({"kc": kc, "vc": vc}[name]), G[f"attn_{name}"])
    for name in ("ks", "vs"):
        np.testing.assert_array_equal(host({"ks": ks, "vs": vs}[name]).view(np.uint32),
                                      G[f"attn_{name}"].view(np.uint32))
    for name, window, pm in (("sliding", 20, 1), ("full", 0, -1)):
        for s_max in (1, 2):
            out, _ = gpu.attention(qi, qb, fq, kc, ks, vc, vs, runs, rows, nq, nkv, hd, window, 4,
                                   page - 1, pm, s_max=s_max)
            torch.cuda.synchronize()
            np.testing.assert_array_equal(host(out), G[f"attn_out_{name}_s{s_max}"],
                                          err_msg=f"{name} s_max={s_max}")
