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
