"""The oracle against golden vectors written by the reference's own codec
(tests/golden/make_golden.py): blob bytes and decoded pages, every preset and
RoPE mode, FP16 (the reference's dtype)."""
import hashlib
import json
from pathlib import Path

import numpy as np
import pytest

from tests.golden.make_golden import case_inputs

GOLDEN = json.loads((Path(__file__).resolve().parent / "golden" / "reference_vectors.json").read_text())
KEYS = {k: int(v, 16) for k, v in GOLDEN["keys"].items()}
AAD = GOLDEN["aad"]


@pytest.mark.parametrize("case", GOLDEN["cases"], ids=lambda c: f"{c['name']}-p{c['preset']}-r{c['rope_mode']}")
def test_oracle_matches_reference_vectors(O, case):
    c = case
    k, v, th = case_inputs(c["tokens"], c["heads"], c["head_dim"], c["rope_dim"], c["mla"],
                           c["pages"], c["seed"])
    blobs = O.egress_batch(k.view(np.uint16), None if v is None else v.view(np.uint16), th,
                           dtype=O.FP16, preset=c["preset"], rope_mode=c["rope_mode"],
                           rope_dim=c["rope_dim"], expected_payload_bytes=c["payload"],
                           tenant_id_hash=AAD["tenant"], model_id_hash=AAD["model"],
                           layer_id=AAD["layer"], head_group_id=AAD["head_group"],
                           base_sequence_nonce=AAD["base_seq"], **KEYS)
    assert hashlib.sha256(blobs.tobytes()).hexdigest() == c["blobs_sha256"]
    if "blobs_hex" in c:
        assert blobs.tobytes().hex() == c["blobs_hex"]
    rc, st, ko, vo = O.ingress_batch(blobs, th, num_tokens=c["tokens"], num_heads=c["heads"],
                                     head_dim=c["head_dim"], rope_dim=c["rope_dim"],
                                     is_mla_single_buffer=c["mla"], dtype=O.FP16,
                                     expected_tenant_hash=AAD["tenant"],
                                     expected_model_hash=AAD["model"],
                                     expected_layer_id=AAD["layer"], **KEYS)
    assert rc == 0
    assert hashlib.sha256(ko.tobytes()).hexdigest() == c["k_sha256"]
    if not c["mla"]:
        assert hashlib.sha256(vo.tobytes()).hexdigest() == c["v_sha256"]
