"""Write tests/golden/moe_small.npz: small seeded MoE blocks (D=FF=256, E=16,
k=4) with their inputs, top-k ids and fp64 outputs from the dense fp64
restatement (oracle.moe.moe_forward_dense64).  Regenerate with
``python tests/golden/make_moe_small.py``."""
import sys
from pathlib import Path

import numpy as np
import torch

sys.path.insert(0, str(Path(__file__).resolve().parents[2]))

from npu_amd import synth
from npu_amd.gguf_types import GGMLQuantizationType as QT
from oracle import moe as OM

CASES = [
    dict(seed=11, T=1, bias=0, norm=0, shared=1, q_gate=int(QT.IQ4_XS), q_down=int(QT.IQ3_XXS)),
    dict(seed=12, T=4, bias=1, norm=1, shared=1, q_gate=int(QT.IQ3_XXS), q_down=int(QT.IQ4_XS)),
    dict(seed=13, T=9, bias=1, norm=0, shared=0, q_gate=int(QT.IQ4_XS), q_down=int(QT.IQ4_XS)),
]


def main() -> None:
    out = {"n_cases": np.int32(len(CASES))}
    for i, c in enumerate(CASES):
        h = synth.host_moe_layer(c["seed"], D=256, FF=256, E=16, k=4, q_gate=c["q_gate"], q_down=c["q_down"],
                                 shared=bool(c["shared"]), bias=bool(c["bias"]), norm=bool(c["norm"]))
        x = synth.host_input(c["seed"] + 100, c["T"], 256, rmsnorm=not c["norm"])
        ol = OM.OracleLayer(h)
        st = {}
        OM.block_forward(torch.from_numpy(x), ol, stages=st)
        y64 = OM.moe_forward_dense64(torch.from_numpy(x), ol).numpy()
        for k, v in c.items():
            out[f"c{i}_{k}"] = np.int32(v)
        out[f"c{i}_x"] = x
        out[f"c{i}_ids"] = st["topk_ids"].numpy().astype(np.int32)
        out[f"c{i}_y64"] = y64
    np.savez_compressed(Path(__file__).with_name("moe_small.npz"), **out)


if __name__ == "__main__":
    main()
