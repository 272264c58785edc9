"""Writes the golden fixtures of this directory (run from the repo root in the build container):

    python tests/golden/make_golden.py

* ``quantizer_constants.json``: for D = 128, the SHA-256 of the fp32 bytes of the
  rotation ``Pi`` for seeds 42 and 43, and the fp32 centroids and boundaries (as
  hex bit patterns) for every supported width.
* ``config1.npz``: BASELINE config 1 (inputs regenerated from seed 0 by
  ``cases.config1_inputs``): the SHA-256 of all packed K/V pages and fp16 norms,
  the packed bytes and norms of pages 0-3, and the fp32 output of the tiled
  compressed-domain operator and the float64 reconstruct operator.

The values come from the oracle (``oracle/``), the CPU restatement of the
reference. The reference keeps no numeric output for this path, so these files
freeze the pinned oracle's results: the CPU tests check that the oracle still
reproduces them, the GPU tests check the HIP append and decode against them.
"""
from __future__ import annotations

import hashlib
import json
import sys
from pathlib import Path

import numpy as np
import torch

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parents[1]))
sys.path.insert(0, str(HERE.parent))

from cases import config1_kv  # noqa: E402
from oracle import attention as oa  # noqa: E402
from oracle.quantizer import get_quantizer  # noqa: E402


def sha(t: torch.Tensor) -> str:
    return hashlib.sha256(t.contiguous().numpy().tobytes()).hexdigest()


def hexbits(t: torch.Tensor) -> list[str]:
    return [f"{int(x) & 0xffffffff:08x}" for x in t.float().view(torch.int32).tolist()]


def quantizer_constants() -> dict:
    out = {"head_dim": 128, "pi_sha256": {}, "codebooks": {}}
    for seed in (42, 43):
        out["pi_sha256"][str(seed)] = sha(get_quantizer(4, 128, seed).Pi)
    for bw in (2, 3, 4, 5, 6, 8):
        tq = get_quantizer(bw, 128, 42)
        out["codebooks"][str(bw)] = {"centroids": hexbits(tq.centroids), "boundaries": hexbits(tq.boundaries)}
    return out


def config1() -> dict:
    torch.set_num_threads(1)                     # one summation order for the CPU GEMMs
    q, _, _, kv = config1_kv()
    scale = oa.default_scale(128)
    out = oa.tiled_compressed_attention(q, kv, scale)
    f64 = oa.reconstruct_attention_f64(q, kv, scale)
    return {
        "sha_k_pages": sha(kv.k_pages), "sha_v_pages": sha(kv.v_pages),
        "sha_k_norms": sha(kv.k_norms.view(torch.int16)), "sha_v_norms": sha(kv.v_norms.view(torch.int16)),
        "k_pages_0_4": kv.k_pages[:4].numpy(), "v_pages_0_4": kv.v_pages[:4].numpy(),
        "k_norms_0_4": kv.k_norms[:4].view(torch.int16).numpy(), "v_norms_0_4": kv.v_norms[:4].view(torch.int16).numpy(),
        "out_tiled_f32": out.numpy(), "out_f64": f64.numpy(),
    }


def main() -> None:
    (HERE / "quantizer_constants.json").write_text(json.dumps(quantizer_constants(), indent=1) + "\n")
    c1 = config1()
    np.savez(HERE / "config1.npz", **{k: (np.array(v) if isinstance(v, str) else v) for k, v in c1.items()})
    print("wrote", HERE / "quantizer_constants.json", HERE / "config1.npz")


if __name__ == "__main__":
    main()
