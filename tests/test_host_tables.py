"""Host-side tables the product builds itself, pinned against the reference.

ythip_rope_tables (libythip.so, host code) is what the Qwen3 runner uploads as
its cos/sin tables. The reference builds them in RoPECache::precompute
(example/qwen3/src/qwen3.cpp:161-175) with float powf / cosf / sinf; the
fixture holds the SHA-256 of the reference's own [4096, 128] tables at
theta 1e6 and five of their rows, written by the compiled reference."""
from __future__ import annotations

import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))


def _fixture():
    return np.load(os.path.join(HERE, "golden", "reference_small.npz"))


def test_product_rope_tables_bit_identical_to_reference():
    from tests.golden import cases
    from ytensor_amd.qwen3 import rope_tables
    g = _fixture()
    c, s = rope_tables(128, 4096, 1e6)
    assert cases.digest(c) == str(g["rope_cos_sha256"])
    assert cases.digest(s) == str(g["rope_sin_sha256"])
    assert np.array_equal(c[[0, 1, 7, 511, 4095]].view(np.uint32), g["rope_cos_rows"].view(np.uint32))


def test_product_rope_tables_closed_form():
    """What the mathematics fixes: row 0 is cos 1 / sin 0; both halves are equal;
    cos^2 + sin^2 = 1; column 0 has frequency 1 (angle = t), so row t column 0
    is cos(t) to float accuracy."""
    from ytensor_amd.qwen3 import rope_tables
    c, s = rope_tables(64, 300, 10000.0)
    assert np.all(c[0] == 1.0) and np.all(s[0] == 0.0)
    assert np.array_equal(c[:, :32], c[:, 32:]) and np.array_equal(s[:, :32], s[:, 32:])
    assert np.abs(c.astype(np.float64) ** 2 + s.astype(np.float64) ** 2 - 1).max() < 1e-6
    t = np.arange(300, dtype=np.float64)
    assert np.abs(c[:, 0] - np.cos(t)).max() < 1e-5
    # column i has frequency theta^(-2i/dim): column 16 of dim 64 is theta^-0.5 = 0.01
    assert np.abs(s[:, 16] - np.sin(t * 0.01)).max() < 1e-5
