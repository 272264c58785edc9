"""Writes ``reference_constants.json`` from the reference's own quantizer (build container only):

    python tests/golden/make_reference_constants.py [/path/to/reference]

The exact fp32 bits of the rotation ``Pi`` and of the Lloyd-Max codebooks are the
one part of the path that no reference test, stored file or closed form fixes
(every code the quantizer emits depends on them). This script imports the
reference's ``TurboQuantMSE`` (turboquant_kv/cache.py:84-106, which calls
``_lloyd_max_gaussian``, cache.py:62-82) in this container and records, for
D = 128:

* the SHA-256 of the fp32 bytes of ``Pi`` for rotation seeds 42 and 43
  (42 is ``quantizers_for``'s default, packed_backend.py:298-303; 43 is the V
  seed of test_packed_attention.py:60-61);
* the fp32 centroids and boundaries as hex bit patterns for every supported
  width (packing.py:24).

The file holds data only (hashes and bit patterns). ``tests/test_golden.py``
checks the oracle and the product's host-side constants against it on the CPU;
the reference itself is never read at test time or on the GPU box.
"""
from __future__ import annotations

import hashlib
import json
import sys
from pathlib import Path

import torch

HERE = Path(__file__).resolve().parent


def _sha(t: torch.Tensor) -> str:
    return hashlib.sha256(t.detach().cpu().float().contiguous().numpy().tobytes()).hexdigest()


def _hexbits(t: torch.Tensor) -> list[str]:
    return [f"{int(x) & 0xffffffff:08x}" for x in t.detach().cpu().float().view(torch.int32).tolist()]


def main(ref_root: str) -> None:
    torch.set_num_threads(1)   # the QR runs single-threaded, as the oracle's does
    sys.path.insert(0, str(Path(ref_root) / "turboquant_kv"))
    import cache as ref_cache  # noqa: E402  (the reference module, imported here only)

    out = {
        "source": "turboquant_kv/cache.py TurboQuantMSE(bit_width, 128, rotation_seed=seed)",
        "torch": torch.__version__,
        "head_dim": 128,
        "pi_sha256": {},
        "codebooks": {},
    }
    for seed in (42, 43):
        out["pi_sha256"][str(seed)] = _sha(ref_cache.TurboQuantMSE(4, 128, "cpu", rotation_seed=seed).Pi)
    for bw in (2, 3, 4, 5, 6, 8):
        tq = ref_cache.TurboQuantMSE(bw, 128, "cpu", rotation_seed=42)
        out["codebooks"][str(bw)] = {"centroids": _hexbits(tq.centroids), "boundaries": _hexbits(tq.boundaries)}
    path = HERE / "reference_constants.json"
    path.write_text(json.dumps(out, indent=1) + "\n")
    print(f"wrote {path}")


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
