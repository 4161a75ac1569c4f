"""The drama-rs-v1 checkpoint reader (src/model.rs:186-291 layout and checks), on the CPU."""
import json

import numpy as np
import pytest

import checkpoint as C
from ckpt_helpers import torch_layer, write_checkpoint


def test_round_trip_names_dtypes_shapes(tmp_path):
    layers = write_checkpoint(tmp_path, [3, 4], E=8)
    meta = C.read_meta(str(tmp_path))
    tc = meta["config"]["text_config"]
    assert tc["num_hidden_layers"] == 2 and tc["num_experts"] == 8
    for i, L in enumerate(layers):
        got = C.read_layer(str(tmp_path), i, tc)
        np.testing.assert_array_equal(got["gu_q"].numpy(), L["gu_q"])
        np.testing.assert_array_equal(got["d_s"].view(dtype=__import__("torch").int16).numpy().view(np.uint16), L["d_s"])
        np.testing.assert_array_equal(got["router"].view(dtype=__import__("torch").int16).numpy().view(np.uint16),
                                      L["router"])
        np.testing.assert_array_equal(got["nw"].numpy(), L["nw"])


def test_rejects_other_formats(tmp_path):
    write_checkpoint(tmp_path, [1], E=8)
    meta = json.load(open(tmp_path / "drama.json"))
    meta["q4_group"] = 32
    json.dump(meta, open(tmp_path / "drama.json", "w"))
    with pytest.raises(C.CheckpointError, match="unsupported converted format"):
        C.read_meta(str(tmp_path))


def test_rejects_wrong_dtype_and_shape(tmp_path):
    import torch

    layers = write_checkpoint(tmp_path, [2], E=8)
    tc = C.read_meta(str(tmp_path))["config"]["text_config"]
    t = torch_layer(layers[0])
    t["router"] = t["router"].float()
    C.write_layer(str(tmp_path), 0, t)
    with pytest.raises(C.CheckpointError, match=r"layer00\.moe\.router: dtype torch.float32, expected torch.bfloat16"):
        C.read_layer(str(tmp_path), 0, tc)
    t = torch_layer(layers[0])
    t["sd_s"] = t["sd_s"][:, :2].contiguous()
    C.write_layer(str(tmp_path), 0, t)
    with pytest.raises(C.CheckpointError, match=r"layer00\.moe\.shared_down\.s: shape"):
        C.read_layer(str(tmp_path), 0, tc)
    t = torch_layer(layers[0])
    del t["nw"]
    C.write_layer(str(tmp_path), 0, t)
    with pytest.raises(C.CheckpointError, match=r"layer00\.post_norm: not in"):
        C.read_layer(str(tmp_path), 0, tc)


def _fp8_layers(E, n, H=2048, I=512):
    import synth

    return [synth.make_layer(60 + i, E=E, H=H, I=I, fmt="ref", kind="fp8", quick=True) for i in range(n)]


def test_fp8_source_assembles_the_kernel_layouts(tmp_path):
    """Fp8Source reads per-expert e4m3 weights and scale_inv blocks spread over two shards and
    assembles gate_up [E, 2I, H] (gate rows, then up rows), s [E, 2I/128, H/128] and down
    [E, H, I], s [E, H/128, I/128] byte for byte (src/model.rs:406-506)."""
    from ckpt_helpers import write_fp8_source

    E = 4
    layers = _fp8_layers(E, 2)
    write_fp8_source(str(tmp_path), layers, E)
    src = C.Fp8Source(str(tmp_path))
    for li, L in enumerate(layers):
        got = src.layer(li, E, 2048, 512)
        np.testing.assert_array_equal(got["gu_q"].numpy(), L["gu_q"])
        np.testing.assert_array_equal(got["d_q"].numpy(), L["d_q"])
        np.testing.assert_array_equal(got["gu_s"].numpy().view(np.uint32), L["gu_s"].view(np.uint32))
        np.testing.assert_array_equal(got["d_s"].numpy().view(np.uint32), L["d_s"].view(np.uint32))


def test_fp8_source_errors(tmp_path):
    import json

    import torch
    from safetensors.torch import save_file
    from ckpt_helpers import write_fp8_source

    E = 2
    layers = _fp8_layers(E, 1)
    write_fp8_source(str(tmp_path), layers, E, shards=1)
    src = C.Fp8Source(str(tmp_path))
    with pytest.raises(C.CheckpointError, match=r"layers\.1\.mlp\.experts\.0\.gate_proj\.weight not in the checkpoint index"):
        src.layer(1, E, 2048, 512)
    with pytest.raises(C.CheckpointError, match="not a multiple of 128"):
        src.layer(0, E, 2048, 500)
    # a scale tensor with the wrong dtype
    idx = json.load(open(tmp_path / "model.safetensors.index.json"))
    name = "model.language_model.layers.0.mlp.experts.1.down_proj.weight_scale_inv"
    save_file({name: torch.zeros(16, 4, dtype=torch.bfloat16)}, str(tmp_path / "bad.safetensors"))
    idx["weight_map"][name] = "bad.safetensors"
    json.dump(idx, open(tmp_path / "model.safetensors.index.json", "w"))
    with pytest.raises(C.CheckpointError, match=r"down_proj\.weight_scale_inv: torch\.bfloat16 \(16, 4\), expected torch\.float32"):
        C.Fp8Source(str(tmp_path)).layer(0, E, 2048, 512)
    with pytest.raises(C.CheckpointError, match="model.safetensors.index.json"):
        C.Fp8Source(str(tmp_path / "missing"))
