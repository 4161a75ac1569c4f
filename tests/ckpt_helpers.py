"""Synthetic drama-rs-v1 checkpoints (reference formats) written from synth.make_layer."""
import numpy as np

import checkpoint as C
import synth


def torch_layer(L):
    import torch

    def f16(a):
        return torch.from_numpy(np.ascontiguousarray(a).view(np.int16)).view(torch.float16)

    return {"nw": torch.from_numpy(L["nw"].copy()),
            "router": torch.from_numpy(np.ascontiguousarray(L["router"]).view(np.int16)).view(torch.bfloat16),
            "gu_q": torch.from_numpy(L["gu_q"].copy()), "gu_s": f16(L["gu_s"]),
            "d_q": torch.from_numpy(L["d_q"].copy()), "d_s": f16(L["d_s"]),
            "sgu_q": torch.from_numpy(L["sgu_q"].copy()), "sgu_s": f16(L["sgu_s"]),
            "sd_q": torch.from_numpy(L["sd_q"].copy()), "sd_s": f16(L["sd_s"])}


def write_checkpoint(path, seeds, E, H=2048, I=512):
    layers = [synth.make_layer(s, E=E, H=H, I=I, fmt="ref") for s in seeds]
    C.write_meta(str(path), H, E, I, len(layers))
    for i, L in enumerate(layers):
        C.write_layer(str(path), i, torch_layer(L))
    return layers


def write_fp8_source(path, layers, E, H=2048, I=512, shards=2):
    """An original-checkpoint directory in the layout the reference reads block-FP8 experts
    from (src/model.rs:406-506): per-expert gate/up/down e4m3 weights and f32 128 x 128
    scale_inv tensors spread over `shards` safetensors files, indexed by
    model.safetensors.index.json.  `layers` hold the assembled arrays (synth.make_layer with
    kind="fp8", fmt="ref"): gu_q [E, 2I, H], gu_s [E, 2I/128, H/128], d_q [E, H, I],
    d_s [E, H/128, I/128]."""
    import json
    import os

    import torch
    from safetensors.torch import save_file

    B = 128
    files = [dict() for _ in range(shards)]
    wmap = {}
    for li, L in enumerate(layers):
        for ex in range(E):
            pre = f"model.language_model.layers.{li}.mlp.experts.{ex}"
            parts = {"gate_proj": (L["gu_q"][ex, :I], L["gu_s"][ex, :I // B]),
                     "up_proj": (L["gu_q"][ex, I:], L["gu_s"][ex, I // B:]),
                     "down_proj": (L["d_q"][ex], L["d_s"][ex])}
            k = (li * E + ex) % shards
            for part, (w, sc) in parts.items():
                files[k][f"{pre}.{part}.weight"] = torch.from_numpy(np.ascontiguousarray(w)).view(torch.float8_e4m3fn)
                files[k][f"{pre}.{part}.weight_scale_inv"] = torch.from_numpy(np.ascontiguousarray(sc, np.float32))
    for k, tensors in enumerate(files):
        name = f"model-{k + 1:05d}-of-{shards:05d}.safetensors"
        save_file(tensors, os.path.join(path, name))
        wmap.update({t: name for t in tensors})
    with open(os.path.join(path, "model.safetensors.index.json"), "w") as f:
        json.dump({"metadata": {}, "weight_map": wmap}, f)
