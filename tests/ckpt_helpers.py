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
