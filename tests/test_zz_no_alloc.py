"""bq_moe_phase2_down_noalloc (phase 2 on the library's static per-GPU
scratch) against bq_moe_phase2_down (caller workspace), through the C ABI:
bit-identical accum and out on calls in a row, each with fewer tokens than
the one before, so the scratch holds the previous call's rows when the next
starts (the first fills it to within 32 KiB of its size);
sizes past the scratch are rejected before anything is launched."""
import numpy as np
import pytest

from test_gpu_parity import dev, host, route_table

pytestmark = pytest.mark.gpu
ONE = 0x3F80


def _layer_inputs(gpu, O, m, T, seed):
    E, H, I = m["E"], m["H"], m["I"]
    x = O.synth_normal_bf16(seed, 1.0, (T, H))
    idx, w = route_table(O, T, seed=seed + 1)
    xq, xsa = gpu.norm_quant(dev(x), dev(np.full(H, ONE, np.uint16)), 128)
    eo, routes = gpu.build_schedule(dev(idx), dev(w), E)
    bucket = gpu.moe_phase1(xq, xsa, eo, routes, m["Wgu"], E, T, 8, I)
    bi8, bsa = gpu.block_quant(bucket, 64, True)
    return eo, routes, bi8, bsa


def test_noalloc_matches_workspace_entry(gpu, O, moe_model):
    import torch
    m = moe_model
    E, H = m["E"], m["H"]
    # each call smaller than the one before; 279 tokens fill the scratch to
    # within 32 KiB of its 24 MiB (279 * 8 * 2816 * 4 bytes), 279 and 256 take
    # the whole-row combine, 96 and 24 the 256-column one
    for T, seed in ((279, 7), (256, 9), (96, 11), (24, 13)):
        print(f"noalloc phase 2: T={T}", flush=True)
        eo, routes, bi8, bsa = _layer_inputs(gpu, O, m, T, seed)
        acc_ws, out_ws = gpu.moe_phase2(bi8, bsa, eo, routes, m["Wd"], E, T, 8, H)
        acc_na, out_na = gpu.moe_phase2_noalloc(bi8, bsa, eo, routes, m["Wd"], E, T, 8, H)
        torch.cuda.synchronize()
        np.testing.assert_array_equal(host(acc_na), host(acc_ws))
        np.testing.assert_array_equal(host(out_na), host(out_ws))


def test_noalloc_rejects_oversize(gpu, O, moe_model):
    import torch
    m = moe_model
    T = 280   # 280 * 8 * 2816 * 4 bytes > 24 MiB
    d = "cuda"
    bi8 = torch.zeros(T * 8, m["I"], dtype=torch.int8, device=d)
    bsa = torch.zeros(T * 8, m["I"] // 64, dtype=torch.float32, device=d)
    eo = torch.zeros(m["E"] + 1, dtype=torch.int32, device=d)
    routes = torch.zeros(T * 8, 2, dtype=torch.int32, device=d)
    with pytest.raises(gpu.BqError) as e:
        gpu.moe_phase2_noalloc(bi8, bsa, eo, routes, m["Wd"], m["E"], T, 8, m["H"])
    assert e.value.code == 4 and "static scratch" in str(e.value)
