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
    return g


if __name__ == "__main__":
    np.savez_compressed(os.path.join(HERE, "golden.npz"), **make())
    print("wrote", os.path.join(HERE, "golden.npz"))
