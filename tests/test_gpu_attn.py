"""GPU parity of the int8-KV attention (libbq.so through its C ABI) against
the CPU oracle: bq_attn_prep (butterquant_kernels/attention.mojo:474-534,
butterquant/head_prep.mojo:9-92) and bq_sliding_attention /
bq_full_attention (attention.mojo:32-471, kernels/logsum_merge.mojo:29-122).

Bar: bit-exact.  Codes, qi_bias, f_q and the whole K/V caches after the prep;
the bf16 attention output for the same split plan (s_max), which fixes the
f32 merge order on both sides.
"""
import numpy as np
import pytest

from attn_cases import make_case, oracle_attention
from test_attn_oracle import rope_tables
from test_gpu_parity import dev, host

pytestmark = pytest.mark.gpu


def gpu_attention(gpu, c, s_max):
    import torch
    runs = dev(np.ascontiguousarray(c.runs).view(np.int32).reshape(-1, 4))
    out, used = gpu.attention(dev(c.q_i8), dev(c.qi_bias), dev(c.f_q), dev(c.k_cache),
                              dev(c.k_scale), dev(c.v_cache), dev(c.v_scale), runs,
                              dev(c.base_rows), c.num_q, c.num_kv, c.head_dim, c.window,
                              c.page_shift, c.row_mask, c.page_mask, s_max=s_max)
    torch.cuda.synchronize()
    return host(out)


def check(gpu, O, c, s_max):
    print(f"attention T={c.T} nq={c.num_q} nkv={c.num_kv} hd={c.head_dim} window={c.window} "
          f"s_max={s_max}", flush=True)
    got = gpu_attention(gpu, c, s_max)
    ref = oracle_attention(O, c, s_max=s_max)
    np.testing.assert_array_equal(got, ref)
    return got


SHAPES = {
    # the sliding layer at decode: window 1024, head_dim 256, GQA 2, ring of two
    # 1024-row pages per sequence
    "sliding_decode_1": dict(num_q=16, num_kv=8, head_dim=256, page_len=1024, window=1024,
                             seqs=[(3000, 1)]),
    "sliding_decode_16": dict(num_q=16, num_kv=8, head_dim=256, page_len=1024, window=1024,
                              seqs=[(int(p), 1) for p in
                                    np.random.default_rng(0).integers(0, 4000, 16)]),
    "sliding_prefill": dict(num_q=16, num_kv=8, head_dim=256, page_len=1024, window=1024,
                            seqs=[(900, 48), (0, 20)]),
    # the full layer: head_dim 512, GQA 8, unbounded page table
    "full_decode_2": dict(num_q=16, num_kv=2, head_dim=512, page_len=256, window=0,
                          seqs=[(2999, 1), (700, 1)]),
    "full_prefill": dict(num_q=16, num_kv=2, head_dim=512, page_len=256, window=0,
                         seqs=[(0, 40), (300, 9)]),
}


@pytest.mark.parametrize("name", sorted(SHAPES))
@pytest.mark.parametrize("plan", ["auto", 1])
def test_attention_model_shapes(gpu, O, name, plan):
    c = make_case(O, 21, **SHAPES[name])
    w = SHAPES[name].get("window", 0)
    s_max = gpu.attention_splits(c.T, c.num_kv, w if w else int(c.positions.max()) + 1) \
        if plan == "auto" else plan
    check(gpu, O, c, s_max)


@pytest.mark.parametrize("gqa", [1, 2, 4, 8, 16])
@pytest.mark.parametrize("hd", [64, 128, 256, 512])
def test_attention_gqa_head_dims(gpu, O, gqa, hd):
    num_kv = 2 if gqa < 16 else 1
    c = make_case(O, gqa * 7 + hd, num_q=gqa * num_kv, num_kv=num_kv, head_dim=hd, page_len=32,
                  window=0 if hd in (64, 512) else 50, seqs=[(37, 3), (5, 1), (130, 2)])
    check(gpu, O, c, 3)


def test_attention_many_splits(gpu, O):
    # s_max above ceil(L/32)/2: some tokens get up to 64 splits, the merge runs
    # over several batches of 16, and short tokens leave splits unused
    c = make_case(O, 8, num_q=4, num_kv=2, head_dim=128, page_len=64, window=0,
                  seqs=[(2100, 1), (10, 1), (64, 1)])
    check(gpu, O, c, 64)


def test_attention_splits_beyond_one_stage(gpu, O):
    # 282 splits for the long token: the many-split merge stages them in two
    # LDS passes (240 + 42)
    c = make_case(O, 12, num_q=2, num_kv=1, head_dim=64, page_len=64, window=0,
                  seqs=[(9000, 1), (100, 1)])
    check(gpu, O, c, 300)


@pytest.mark.parametrize("gqa,hd", [(1, 64), (2, 128), (2, 256), (4, 128), (8, 64), (8, 256)])
@pytest.mark.parametrize("window,seqs", [
    (40, [(50, 70)]),             # every token past the window start: shifted tile grids
    (40, [(5, 70), (200, 3)]),    # a run straddling pos = window - 1, then a short run
    (0, [(0, 130), (37, 20)]),    # full attention, two runs
])
def test_attention_single_split_groups(gpu, O, gqa, hd, window, seqs):
    # one split per token (s_max = 1): tokens t, t + 16, ... of a run share a
    # wave when their tile grids coincide; the rest run one per pass
    c = make_case(O, gqa * 3 + hd + window, num_q=2 * gqa, num_kv=2, head_dim=hd, page_len=64,
                  window=window, ring_pages=4, seqs=seqs)
    check(gpu, O, c, 1)


def prep_case(O, seed, hd, rope_half, ps, nq, nkv, seqs, page, degree=1, rank=0,
              k_eq_v=False):
    rng = np.random.default_rng(seed)
    T = sum(n for _, n in seqs)
    bf = lambda *shape: O.f32_to_bf16(rng.standard_normal(shape).astype(np.float32) * 2)
    q, k = bf(T, nq * hd), bf(T, nkv * hd)
    v = k if k_eq_v else bf(T, nkv * hd)
    qn = O.f32_to_bf16(rng.uniform(0.5, 1.5, hd).astype(np.float32))
    kn = O.f32_to_bf16(rng.uniform(0.5, 1.5, hd).astype(np.float32))
    maxpos = max(b + n for b, n in seqs)
    cos, sin = rope_tables(maxpos + 1, rope_half)
    runs, rows, buf, off = [], [], 0, 0
    npages = 0
    for b, n in seqs:
        need = ((b + n) // degree) // page + 1
        runs.append((buf, b, off, need))
        rows.extend(range(npages, npages + need))
        npages += need
        buf += n
        off += need
    perm = rng.permutation(npages + 2)
    rows = (perm[np.array(rows)] * page).astype(np.int32)
    slots = (npages + 2) * page
    caches = dict(kc=np.zeros((slots, nkv * hd), np.int8), ks=np.zeros((slots, nkv), np.float32),
                  vc=np.zeros((slots, nkv * hd), np.int8), vs=np.zeros((slots, nkv), np.float32))
    return dict(q=q, k=k, v=v, qn=qn, kn=kn, cos=cos, sin=sin, runs=O.kv_runs(runs), rows=rows,
                shift=int(np.log2(page)), page=page, degree=degree, rank=rank, **caches)


@pytest.mark.parametrize("hd,rope_half,ps,nq,nkv,degree,rank,k_eq_v", [
    (256, 128, 128, 16, 8, 1, 0, False),    # the sliding layer
    (512, 64, 256, 16, 2, 1, 0, True),      # the full layer (K = V projection)
    (512, 64, 256, 16, 2, 2, 1, True),      # cache rank 1 of 2
    (128, 64, 64, 4, 4, 1, 0, False),
    (64, 0, 0, 2, 1, 1, 0, False),          # no RoPE
])
def test_attn_prep(gpu, O, hd, rope_half, ps, nq, nkv, degree, rank, k_eq_v):
    import torch
    p = prep_case(O, hd + nq, hd, rope_half, ps, nq, nkv, [(100, 7), (3, 2), (1500, 1)], 64,
                  degree, rank, k_eq_v)
    print(f"attn_prep hd={hd} rope_half={rope_half} degree={degree}", flush=True)
    g = {n: dev(p[n]) for n in ("kc", "ks", "vc", "vs")}
    runs = dev(np.ascontiguousarray(p["runs"]).view(np.int32).reshape(-1, 4))
    qi, qb, fq = gpu.attn_prep(dev(p["q"]), dev(p["k"]), dev(p["v"]), dev(p["qn"]), dev(p["kn"]),
                               g["kc"], g["ks"], g["vc"], g["vs"], dev(p["cos"]), dev(p["sin"]),
                               runs, dev(p["rows"]), nq, nkv, hd, rope_half, ps, p["shift"],
                               p["page"] - 1, -1, cache_degree=degree, rank=rank)
    torch.cuda.synchronize()
    rqi, rqb, rfq = O.attn_prep(p["q"], p["k"], p["v"], p["qn"], p["kn"], p["kc"], p["ks"],
                                p["vc"], p["vs"], p["cos"], p["sin"], p["runs"], p["rows"], nq,
                                nkv, hd, rope_half, ps, p["shift"], p["page"] - 1, -1,
                                cache_degree=degree, rank=rank)
    np.testing.assert_array_equal(host(qi), rqi)
    np.testing.assert_array_equal(host(qb).view(np.uint32), rqb.view(np.uint32))
    np.testing.assert_array_equal(host(fq).view(np.uint32), rfq.view(np.uint32))
    for n in ("kc", "ks", "vc", "vs"):
        np.testing.assert_array_equal(host(g[n]).view(np.uint8), p[n].view(np.uint8))


def test_prep_then_attention(gpu, O):
    """The layer's two calls back to back: prep fills the cache, attention
    reads it (sliding, decode batch of 3 sequences continuing from
    prefilled caches)."""
    import torch
    hd, nq, nkv, page = 256, 16, 8, 64
    p = prep_case(O, 99, hd, 128, 128, nq, nkv, [(0, 70), (0, 33), (0, 5)], page)
    runs = dev(np.ascontiguousarray(p["runs"]).view(np.int32).reshape(-1, 4))
    g = {n: dev(p[n]) for n in ("kc", "ks", "vc", "vs")}
    qi, qb, fq = gpu.attn_prep(dev(p["q"]), dev(p["k"]), dev(p["v"]), dev(p["qn"]), dev(p["kn"]),
                               g["kc"], g["ks"], g["vc"], g["vs"], dev(p["cos"]), dev(p["sin"]),
                               runs, dev(p["rows"]), nq, nkv, hd, 128, 128, p["shift"], page - 1,
                               -1)
    out, s_max = gpu.attention(qi, qb, fq, g["kc"], g["ks"], g["vc"], g["vs"], runs,
                               dev(p["rows"]), nq, nkv, hd, 48, p["shift"], page - 1, -1)
    torch.cuda.synchronize()
    rqi, rqb, rfq = O.attn_prep(p["q"], p["k"], p["v"], p["qn"], p["kn"], p["kc"], p["ks"],
                                p["vc"], p["vs"], p["cos"], p["sin"], p["runs"], p["rows"], nq,
                                nkv, hd, 128, 128, p["shift"], page - 1, -1)
    ref = O.flash_attention(rqi, rqb, rfq, p["kc"], p["ks"], p["vc"], p["vs"], p["runs"],
                            p["rows"], nq, nkv, hd, 48, p["shift"], page - 1, -1, s_max=s_max)
    np.testing.assert_array_equal(host(out), ref)
