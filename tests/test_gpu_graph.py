"""HIP-graph replays of a decoder layer's launches equal the eager calls, bit
for bit, on every replay (the benchmarks time graph replays): norm-quant,
q/k/v, block-quant + o_proj, and the FFN's prep, gate/up and down with the
dense MLP in the experts' launches.  Between replays the outputs are
overwritten and other eager work runs; 16 tokens take the one-workgroup MoE
prep, 32 tokens the spread form with its per-stream completion counter."""
import numpy as np
import pytest

from test_gpu_parity import ONE, dev, weight

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("T", [16, 32])
def test_decoder_layer_graph_replays(gpu, O, T):
    import torch
    E, k, H, I, DI, QN, KVN, B = 16, 4, 1024, 128, 192, 512, 256, 256
    Wgu = weight(gpu, O, E * 2 * I, H, 128, seed=51)[2]
    Wd = weight(gpu, O, E * H, I, 64, seed=52)[2]
    Wq, Wk, Wv = (weight(gpu, O, n, H, 128, seed=sd)[2] for n, sd in ((QN, 53), (KVN, 54), (KVN, 55)))
    Wo = weight(gpu, O, H, QN, B, seed=56)[2]
    Wg, Wu = (weight(gpu, O, DI, H, 128, seed=sd)[2] for sd in (57, 58))
    Wdd = weight(gpu, O, H, DI, 64, seed=59)[2]
    x = dev(O.synth_normal_bf16(60 + T, 1.0, (T, H)))
    attn = dev(O.synth_normal_bf16(61 + T, 1.0, (T, QN)))
    logits = dev(O.synth_normal_f32(62 + T, 1.0, (T, E)))
    gamma = dev(np.full(H, ONE, np.uint16))
    gamma2 = dev(O.f32_to_bf16(O.synth_normal_f32(63, 0.3, (H,)) + 1.0))
    d = "cuda"
    e = lambda *shape, dt=torch.bfloat16: torch.empty(*shape, dtype=dt, device=d)
    out = dict(
        xq=e(T, H, dt=torch.int8), xsa=e(T, dt=torch.float32),
        q=e(T, QN), k=e(T, KVN), v=e(T, KVN),
        oq=e(T, QN, dt=torch.int8), osa=e(T, QN // B, dt=torch.float32), o=e(T, H),
        idx=e(T, k, dt=torch.int32), w=e(T, k, dt=torch.float32), eo=e(E + 1, dt=torch.int32),
        routes=torch.zeros(T * k, 2, dtype=torch.int32, device=d),
        mq=e(T, H, dt=torch.int8), msa=e(T, dt=torch.float32),
        dq=e(T, H, dt=torch.int8), dsa=e(T, dt=torch.float32),
        bi8=e(T * k, I, dt=torch.int8), bsa=e(T * k, I // 64, dt=torch.float32),
        gq=e(T, DI, dt=torch.int8), gsa=e(T, DI // 64, dt=torch.float32),
        acc=e(T, H, dt=torch.float32), mo=e(T, H), do=e(T, H))
    ws = torch.empty(max(gpu.moe_phase2_workspace_size(T, k, H), 256), dtype=torch.uint8, device=d)

    def layer():
        gpu.norm_quant(x, gamma, 128, out=(out["xq"], out["xsa"]))
        gpu.qkv(out["xq"], out["xsa"], Wq, Wk, Wv, outs=(out["q"], out["k"], out["v"]))
        gpu.block_quant(attn, B, False, out=(out["oq"], out["osa"]))
        gpu.block_linear(out["oq"], out["osa"], Wo, B, out=out["o"])
        gpu.ffn_prep(logits, x, gamma, gamma2, k, None, 128,
                     out=tuple(out[n] for n in ("idx", "w", "eo", "routes", "mq", "msa", "dq", "dsa")))
        gpu.ffn_gate_up(out["mq"], out["msa"], out["eo"], out["routes"], Wgu, E, T, k, I,
                        out["dq"], out["dsa"], Wg, Wu,
                        out=(out["bi8"], out["bsa"], out["gq"], out["gsa"]))
        gpu.ffn_down(out["bi8"], out["bsa"], out["eo"], out["routes"], Wd, E, T, k, H, out["gq"],
                     out["gsa"], Wdd, 64, workspace=ws, out=(out["acc"], out["mo"], out["do"]))

    layer()
    torch.cuda.synchronize()
    ref = {n: t.clone() for n, t in out.items()}
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        layer()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        layer()
    torch.cuda.synchronize()
    other = dev(O.synth_normal_bf16(64, 1.0, (T, H)))
    for rep in range(4):
        for t in out.values():  # every output is rewritten by the replay
            t.view(torch.uint8).fill_(0xA5)
        gpu.norm_quant(other, gamma2, 128)  # eager work between replays
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        for n, t in out.items():
            assert torch.equal(t.view(torch.uint8), ref[n].view(torch.uint8)), (rep, n)
