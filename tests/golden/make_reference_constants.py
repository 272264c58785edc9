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
  width (packing.py:24);
* the SHA-256 of ``Pi`` as the reference builds it on the thread counts 1, 2, 4
  and 8, and at this container's default thread count (``pi_sha256_by_threads``,
  ``default_threads``). ``TurboQuantMSE`` (cache.py:92-97) does not pin the
  number of threads its fp32 ``torch.linalg.qr`` runs on, and the bits of ``Pi``
  depend on it: the product and the oracle reproduce the single-threaded
  construction (``pi_sha256``), which a multi-core host's reference does not.

The file holds data only (hashes and bit patterns). ``tests/test_golden.py``
checks the oracle and the product's host-side constants against it on the CPU;
the reference itself is never read at test time or on the GPU box.

It also writes ``winnow_amd/rotations_d128.npz``: the fp32 bits of the reference's
single-threaded ``Pi`` at D = 128 for seeds 42 and 43. The fp32 QR's bits depend
on the host's CPU and thread count, so the product and the oracle load these
standard rotations instead of rebuilding them, and every host encodes with the
same ``Pi`` (``tests/test_golden.py`` pins the file to the SHAs above).
"""
from __future__ import annotations

import hashlib
import json
import sys
from pathlib import Path

import numpy as np
import torch

HERE = Path(__file__).resolve().parent


def _sha(t: torch.Tensor) -> str:
    return hashlib.sha256(t.detach().cpu().float().contiguous().numpy().tobytes()).hexdigest()


def _hexbits(t: torch.Tensor) -> list[str]:
    return [f"{int(x) & 0xffffffff:08x}" for x in t.detach().cpu().float().view(torch.int32).tolist()]


def main(ref_root: str) -> None:
    default_threads = torch.get_num_threads()
    sys.path.insert(0, str(Path(ref_root) / "turboquant_kv"))
    import cache as ref_cache  # noqa: E402  (the reference module, imported here only)

    out = {
        "source": "turboquant_kv/cache.py TurboQuantMSE(bit_width, 128, rotation_seed=seed)",
        "torch": torch.__version__,
        "head_dim": 128,
        "pi_sha256": {},
        "default_threads": default_threads,
        "pi_sha256_by_threads": {},
        "codebooks": {},
    }
    for threads in sorted({1, 2, 4, 8, default_threads}):
        torch.set_num_threads(threads)
        out["pi_sha256_by_threads"][str(threads)] = {
            str(seed): _sha(ref_cache.TurboQuantMSE(4, 128, "cpu", rotation_seed=seed).Pi) for seed in (42, 43)}
    torch.set_num_threads(1)   # the construction the product and the oracle reproduce
    rot = {}
    for seed in (42, 43):
        pi = ref_cache.TurboQuantMSE(4, 128, "cpu", rotation_seed=seed).Pi.detach().float().contiguous()
        out["pi_sha256"][str(seed)] = _sha(pi)
        rot[f"pi_{seed}"] = pi.numpy()
    rot_path = HERE.parents[1] / "winnow_amd" / "rotations_d128.npz"
    np.savez(rot_path, **rot)
    print(f"wrote {rot_path}")
    for bw in (2, 3, 4, 5, 6, 8):
        tq = ref_cache.TurboQuantMSE(bw, 128, "cpu", rotation_seed=42)
        out["codebooks"][str(bw)] = {"centroids": _hexbits(tq.centroids), "boundaries": _hexbits(tq.boundaries)}
    path = HERE / "reference_constants.json"
    path.write_text(json.dumps(out, indent=1) + "\n")
    print(f"wrote {path}")


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
