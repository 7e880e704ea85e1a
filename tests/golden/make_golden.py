"""Generate tests/golden/golden.npz: small known-answer vectors of the
butterquant hot path computed by the pinned CPU oracle (oracle/bq_oracle.c).

The reference (Mojo) holds no golden vectors for this path and cannot be run
here, so these fixtures are produced by the oracle after it passes
tests/test_oracle_pins.py.  They freeze the oracle's outputs (regression pin)
and give the GPU tests size-small exact targets.

    python tests/golden/make_golden.py
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(HERE, "..", "..", "oracle"))
import oracle as O  # noqa: E402

ONE = 0x3F80  # bf16 1.0


def make():
    g = {}
    for B in (16, 32, 64, 128, 256, 512):
        x = O.synth_normal_f32(100 + B, 1.0, (2, B))
        g[f"fwht{B}_in"] = x
        g[f"fwht{B}_out"] = O.fwht_rows(x, B)

    xq = np.array([127, 2.5, 3.5, -2.5, -0.5, 0.5, 1.5, 63.5, -63.5, 0.0], np.float32)
    q, s = O.quant_segment(xq, False)
    g["quant_in"], g["quant_codes"], g["quant_scale"] = xq, q, np.float32(s)

    w = O.synth_normal_bf16(0, 0.02, (64, 256))
    wq, ws = O.rotate_and_quant(O.bf16_to_f32(w), 128)
    wqb, wsb = O.rotate_and_quant(O.bf16_to_f32(w), 64, per_block=True)
    g["rq_w"], g["rq_codes"], g["rq_scales"] = w, wq, ws
    g["rq_codes_pb64"], g["rq_scales_pb64"] = wqb, wsb

    pw = (np.arange(64 * 128) % 251 - 125).astype(np.int8).reshape(64, 128)
    pk, pcs = O.pack_and_colsum(pw)
    pk2, pcs2 = O.pack_and_colsum(pw, 64, False)
    g["pack_w"], g["pack_vnni"], g["pack_colsum"], g["pack_colsum_b64"] = pw, pk, pcs, pcs2

    x = O.synth_normal_bf16(1, 1.0, (4, 512))
    gam = O.f32_to_bf16(np.linspace(0.5, 1.5, 512).astype(np.float32))
    nq, nsa = O.norm_quant(x, gam, 128)
    g["nq_x"], g["nq_gamma"], g["nq_codes"], g["nq_sa"] = x, gam, nq, nsa

    xb = O.synth_normal_bf16(2, 1.0, (4, 704))
    bq_, bsa = O.block_quant(xb, 64, True)
    g["bq_x"], g["bq_codes"], g["bq_sa"] = xb, bq_, bsa

    # per-row linear (M=3, N=64, K=256) and per-block linear (B=64)
    lp, lcs = O.pack_and_colsum(wq)
    xl = O.synth_normal_bf16(3, 1.0, (3, 256))
    lxq, lsa = O.norm_quant(xl, np.full(256, ONE, np.uint16), 128)
    lob, lof = O.linear(lxq, lsa, lp, ws, lcs, 64)
    g["lin_xq"], g["lin_sa"], g["lin_out_bf16"], g["lin_out_f32"] = lxq, lsa, lob, lof
    wq64, ws64 = O.rotate_and_quant(O.bf16_to_f32(w), 64)
    bp, bcs = O.pack_and_colsum(wq64, 64, False)
    bxq, bxs = O.block_quant(O.synth_normal_bf16(4, 1.0, (3, 256)), 64, True)
    bob, bof = O.block_linear(bxq, bxs, bp, ws64, bcs, 64, 64)
    g["blin_codes"], g["blin_scales"] = wq64, ws64
    g["blin_xq"], g["blin_sa"], g["blin_out_bf16"], g["blin_out_f32"] = bxq, bxs, bob, bof

    # tiny MoE: T=6 tokens, E=4 experts, top-2, hidden 128, inter 64
    T, E, k, H, I = 6, 4, 2, 128, 64
    logits = O.synth_normal_f32(5, 1.0, (T, E))
    idx, rw = O.route_topk_softmax(logits, k)
    eo, routes = O.build_schedule(idx, rw, E)
    gu = O.synth_normal_bf16(6, 0.02, (E * 2 * I, H))
    gq, gs = O.rotate_and_quant(O.bf16_to_f32(gu), 128)
    gp, gcs = O.pack_and_colsum(gq)
    dn = O.synth_normal_bf16(7, 0.02, (E * H, I))
    dq, ds = O.rotate_and_quant(O.bf16_to_f32(dn), 64)
    dp, dcs = O.pack_and_colsum(dq, 64, False)
    xm = O.synth_normal_bf16(8, 1.0, (T, H))
    mxq, mxs = O.norm_quant(xm, np.full(H, ONE, np.uint16), 128)
    bucket = O.moe_phase1(mxq, mxs, eo, routes, gp, gs, gcs, I)
    bkq, bks = O.block_quant(bucket, 64, True)
    acc, out = O.moe_phase2(bkq, bks, eo, routes, T, dp, ds, dcs, H)
    g.update(moe_logits=logits, moe_idx=idx, moe_w=rw, moe_eo=eo,
             moe_route_token=routes["token"].copy(), moe_route_weight=routes["weight"].copy(),
             moe_gq=gq, moe_gs=gs, moe_dq=dq, moe_ds=ds, moe_x=xm, moe_xq=mxq, moe_xsa=mxs,
             moe_bucket=bucket, moe_bucket_i8=bkq, moe_bucket_sa=bks, moe_accum=acc,
             moe_out=out)

    # router: logits (T=3, E=8, H=256) and top-2 softmax with a per-expert scale
    rx = O.synth_normal_bf16(9, 1.0, (3, 256))
    rproj = O.synth_normal_bf16(10, 0.05, (8, 256))
    rsc = O.f32_to_bf16(np.linspace(0.5, 1.5, 256).astype(np.float32))
    rlog = O.router_logits(rx, rproj, rsc)
    pes = O.f32_to_bf16(np.linspace(0.75, 1.25, 8).astype(np.float32))
    ridx, rwt = O.route_topk_softmax(rlog, 2, pes)
    g.update(router_x=rx, router_proj=rproj, router_scale=rsc, router_logits=rlog,
             router_pes=pes, router_idx=ridx, router_w=rwt)

    # vocabulary head: V=160, H=256, B=128, two rows (one greedy), and the
    # embedding rows of the same table
    rng = np.random.default_rng(11)
    hw = rng.integers(-127, 128, (160, 256), dtype=np.int8)
    hws = (rng.random((160, 2)) / 127 / 30).astype(np.float32)
    hx = O.synth_normal_bf16(12, 1.0, (2, 256))
    hxq, hxs = O.norm_quant(hx, np.full(256, ONE, np.uint16), 128, per_block=True)
    hp = O.sampling_params(2, temperature=[0.8, 1.0], top_k=[20, 0], seed=[7, 8], n_keep=[16, 4],
                           greedy=[False, True])
    hout = O.flash_sample(hxq, hxs, hw, hws, hp)
    etok = np.array([0, 159, 42, 42], np.int32)
    emb = O.embed_lookup(etok, hw, hws, 128, scale=O.embed_scale(2816))
    g.update(head_w=hw, head_ws=hws, head_xq=hxq, head_xsa=hxs,
             head_params=np.frombuffer(hp.tobytes(), np.uint8),
             head_outcome=np.frombuffer(hout.tobytes(), np.uint8), embed_tokens=etok, embed_out=emb)

    # int8-KV attention: prep of 5 tokens (two runs) into a 6-page cache of
    # 16 rows (head_dim 128, 4 q / 2 kv heads, RoPE on 64 of 64 pairs), then
    # sliding (window 20) and full attention with one and two splits
    nq, nkv, hd, page = 4, 2, 128, 16
    ax = lambda seed, n: O.synth_normal_bf16(seed, 1.0, (5, n))
    aq, ak, av = ax(13, nq * hd), ax(14, nkv * hd), ax(15, nkv * hd)
    qn = O.f32_to_bf16(np.linspace(0.5, 1.5, hd).astype(np.float32))
    kn = O.f32_to_bf16(np.linspace(1.5, 0.5, hd).astype(np.float32))
    ang = np.arange(64)[:, None] * (1.0 / 10000.0 ** (np.arange(64) / 64.0))[None, :]
    cos, sin = np.cos(ang).astype(np.float32), np.sin(ang).astype(np.float32)
    runs = O.kv_runs([(0, 14, 0, 2), (3, 7, 2, 1)])  # positions 14-16 and 7-8: pages 0, 1
    rows = np.array([2 * page, 5 * page, 0], np.int32)
    crng = np.random.default_rng(16)
    kc = crng.integers(-127, 128, (6 * page, nkv * hd), dtype=np.int8)
    vc = crng.integers(-127, 128, (6 * page, nkv * hd), dtype=np.int8)
    ks = crng.uniform(1, 6, (6 * page, nkv)).astype(np.float32)
    vs = crng.uniform(0.5, 3, (6 * page, nkv)).astype(np.float32)
    g.update(attn_q=aq, attn_k=ak, attn_v=av, attn_qn=qn, attn_kn=kn, attn_cos=cos,
             attn_sin=sin, attn_runs=np.frombuffer(runs.tobytes(), np.int32).reshape(-1, 4),
             attn_rows=rows, attn_kc_in=kc.copy(), attn_vc_in=vc.copy(), attn_ks_in=ks.copy(),
             attn_vs_in=vs.copy())
    qi, qb, fq = O.attn_prep(aq, ak, av, qn, kn, kc, ks, vc, vs, cos, sin, runs, rows, nq, nkv,
                             hd, 64, 64, 4, page - 1, -1)
    g.update(attn_qi=qi, attn_qb=qb, attn_fq=fq, attn_kc=kc, attn_ks=ks, attn_vc=vc, attn_vs=vs)
    for name, window, pm in (("sliding", 20, 1), ("full", 0, -1)):
        for s_max in (1, 2):
            g[f"attn_out_{name}_s{s_max}"] = O.flash_attention(
                qi, qb, fq, kc, ks, vc, vs, runs, rows, nq, nkv, hd, window, 4, page - 1, pm,
                s_max=s_max, min_split=32)
    return g


if __name__ == "__main__":
    np.savez_compressed(os.path.join(HERE, "golden.npz"), **make())
    print("wrote", os.path.join(HERE, "golden.npz"))
