"""The product's quantizer constants, built on the GPU box's own host, against the fixture.

``winnow_amd.quantizer.get_quantizer`` builds ``Pi`` (seeded ``torch.randn`` and a
single-threaded fp32 ``torch.linalg.qr`` with the sign fix, turboquant_kv/cache.py:92-97)
and the Lloyd-Max codebook (cache.py:62-82) on the host of the machine it runs on, then
moves them to the device. Every code the append writes depends on those bits, so the
bits the GPU box builds must be the ones committed in
``tests/golden/quantizer_constants.json`` (which equal the reference's single-threaded
construction, ``reference_constants.json``). The CPU suite checks the same on the build
container; this runs on the GPU box.

The fp32 QR rounds differently on the GPU box's CPU than on the build container's, so
the standard rotations (head_dim 128, seeds 42 and 43) ship as data
(``winnow_amd/rotations_d128.npz``) and are loaded, not rebuilt; other head dims run
the QR on the host, and there the product and the oracle must agree with each other.
"""
from __future__ import annotations

import hashlib
import json
from pathlib import Path

import pytest
import torch

pytestmark = pytest.mark.gpu

GOLDEN = Path(__file__).resolve().parent / "golden"


@pytest.fixture(scope="module")
def constants():
    return json.loads((GOLDEN / "quantizer_constants.json").read_text())


def _sha(t: torch.Tensor) -> str:
    return hashlib.sha256(t.detach().cpu().float().contiguous().numpy().tobytes()).hexdigest()


def _hex(t: torch.Tensor) -> list[str]:
    return [f"{int(x) & 0xffffffff:08x}" for x in t.detach().cpu().float().view(torch.int32).tolist()]


@pytest.mark.parametrize("seed", [42, 43])
def test_product_pi_bits_on_this_host(constants, seed):
    from winnow_amd.quantizer import get_quantizer
    tq = get_quantizer(4, 128, "cuda", seed)
    assert tq.Pi.device.type == "cuda"
    assert _sha(tq.Pi) == constants["pi_sha256"][str(seed)]


@pytest.mark.parametrize("bw", [2, 3, 4, 5, 6, 8])
def test_product_codebook_bits_on_this_host(constants, bw):
    from winnow_amd.quantizer import get_quantizer
    tq = get_quantizer(bw, 128, "cuda", 42)
    want = constants["codebooks"][str(bw)]
    assert _hex(tq.centroids) == want["centroids"]
    assert _hex(tq.boundaries) == want["boundaries"]


@pytest.mark.parametrize("D,seed", [(128, 42), (128, 43), (64, 42), (32, 43)])
def test_product_and_oracle_use_the_same_rotation_here(D, seed):
    from oracle.quantizer import qr_rotation, rotation
    from winnow_amd.quantizer import get_quantizer
    assert _sha(get_quantizer(4, D, "cuda", seed).Pi) == _sha(rotation(D, seed))
    if D != 128:
        assert _sha(rotation(D, seed)) == _sha(qr_rotation(D, seed))
