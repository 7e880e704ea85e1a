"""GPU check of the on-disk -> device weight path (bq_load_quantized):
int8 codes + f32 scales read from safetensors shards, validated, copied and
re-tiled; the codes read back through bq_weight_unpack bit-exact, the scales
byte-identical."""
import numpy as np
import pytest

from test_gpu_parity import host

pytestmark = pytest.mark.gpu


def test_load_quantized(gpu, tmp_path):
    import torch
    from safetensors.numpy import save_file
    rng = np.random.default_rng(3)
    n, k, B = 96, 256, 128
    w = rng.integers(-128, 128, (n, k), dtype=np.int8)
    s = rng.random(n).astype(np.float32)
    wb = rng.integers(-128, 128, (2, 48, k), dtype=np.int8)   # [experts, rows, k]
    sb = rng.random((2, 48, k // B)).astype(np.float32)
    save_file({"proj": w, "experts": wb}, str(tmp_path / "model-00001.safetensors"))
    save_file({"proj.scale": s, "experts.scale": sb, "bad.scale": s.astype(np.float16),
               "bad": w}, str(tmp_path / "model-00002.safetensors"))
    files = [gpu.SafetensorsFile(str(tmp_path / f"model-0000{i}.safetensors")) for i in (1, 2)]
    # a staging buffer of two strips forces three chunks
    staging = torch.empty(2 * 16 * k, dtype=torch.int8, device="cuda")
    W = gpu.load_quantized(files, "proj", n, k, staging=staging)
    np.testing.assert_array_equal(host(gpu.unpack(W.data, n, k)).reshape(n, k), w)
    np.testing.assert_array_equal(host(W.scale), s)
    # 3-D experts tensor folded to rows, per-block scales
    E = gpu.load_quantized(files, "experts", 96, k, scale_cols=k // B)
    np.testing.assert_array_equal(host(gpu.unpack(E.data, 96, k)).reshape(96, k), wb.reshape(96, k))
    np.testing.assert_array_equal(host(E.scale), sb.reshape(96, k // B))
    with pytest.raises(gpu.BqError, match="dtype mismatch|dtype or shape"):
        gpu.load_quantized(files, "bad", n, k)
    with pytest.raises(gpu.BqError, match="shape mismatch"):
        gpu.load_quantized(files, "proj", n, 128)
    with pytest.raises(gpu.BqError, match="missing tensor"):
        gpu.load_quantized(files, "absent", n, k)
