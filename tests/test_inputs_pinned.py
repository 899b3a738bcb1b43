"""The seeded inputs every configuration is tested and benchmarked on are
pinned: SHA-256 of the fp16/bf16 bit patterns generated on the CPU (seed
1234 + 100003*i, input_data.py:11-12), and C1 equal to the committed golden
fixture.  A change of torch's generator or of the seeding shows up here
rather than as silently different test data."""
from __future__ import annotations

import hashlib
import os

import numpy as np
import pytest
import torch

from helpers import make_config

HERE = os.path.dirname(os.path.abspath(__file__))

PINNED = {
    "C1": "b518f774ca6ff9ca2d1cd7e0897b7d71c0adab14760f0c252cb8da686fd5b366",
    "C2": "f8c57fb58a1545ef49fd717b8f5c373bfed9aa59e61b9482fd8a2339d256afcd",
    "C5r": "0918b47e862175b2df6a713a185286ce048d08af5d74a35246c03b27881dba9b",
}


@pytest.mark.parametrize("name", sorted(PINNED))
def test_config_inputs_sha256(name):
    q, k, v, _, _ = make_config(name)
    h = hashlib.sha256()
    for t in (q, k, v):
        h.update(t.contiguous().view(-1).view(torch.int16).numpy().tobytes())
    assert h.hexdigest() == PINNED[name]


def test_c1_inputs_equal_golden_fixture():
    z = np.load(os.path.join(HERE, "golden", "c1_golden.npz"))
    q, k, v, _, _ = make_config("C1")
    for t, key in ((q, "q_f16"), (k, "k_f16"), (v, "v_f16")):
        assert np.array_equal(t.view(torch.int16).numpy().view(np.uint16), z[key].view(np.uint16))
