"""CPU tests of the benchmark input modes (fa_bench/input_data.py), which
follow the four modes of the reference's benchmark/python/input_data.py."""
from __future__ import annotations

import math

import pytest
import torch

from fa_bench.input_data import case_seed, generate_qkv


def _gen(mode, shape=(2, 3, 40, 64), dtype=torch.float32, **kw):
    B, H, N, D = shape
    return generate_qkv(batch_size=B, n_heads=H, seq_len=N, d_head=D, dtype=dtype, device="cpu",
                        input_mode=mode, **kw)


def test_case_seed():
    assert case_seed(1234, 0) == 1234
    assert case_seed(1234, 2) == 1234 + 2 * 100003


def test_random_is_seeded_and_matches_configs():
    q1, k1, v1, p = _gen("random", seed=5, case_index=1)
    q2, k2, v2, _ = _gen("random", seed=5, case_index=1)
    q3, _, _, _ = _gen("random", seed=5, case_index=2)
    assert p is None
    assert torch.equal(q1, q2) and torch.equal(k1, k2) and torch.equal(v1, v2)
    assert not torch.equal(q1, q3)
    # qk_sigma scales Q and K only
    qs, ks, vs, _ = _gen("random", seed=5, case_index=1, qk_sigma=3.0)
    assert torch.allclose(qs, 3 * q1) and torch.allclose(ks, 3 * k1) and torch.equal(vs, v1)


def test_structured_closed_form():
    q, k, v, _ = _gen("structured")
    for (b, h, n, d) in [(0, 0, 0, 0), (1, 2, 39, 63), (1, 0, 17, 5)]:
        assert q[b, h, n, d].item() == pytest.approx(
            math.sin((n + 1) * (h + 1) / 17.0) + 0.01 * d + 0.05 * b, abs=1e-6)
        assert k[b, h, n, d].item() == pytest.approx(
            math.cos((n + 1) * (h + 1) / 19.0) + 0.02 * d + 0.03 * b, abs=1e-6)
        assert v[b, h, n, d].item() == pytest.approx(
            math.sin((d + 1) * (h + 1) / 23.0) + 0.001 * n + 0.02 * b, abs=1e-6)


def test_stress_scales_and_outliers():
    q, k, v, _ = _gen("stress", shape=(2, 4, 512, 128), seed=3)
    # N(0, 32^2) bulk with a ~1e-3 fraction of +256 outliers on Q
    assert 28 < q.float().std().item() < 40
    big = (q > 200).float().mean().item()
    assert 2e-4 < big < 3e-3
    assert (k < -200).float().mean().item() > 2e-4
    assert 14 < v.float().std().item() < 20


@pytest.mark.parametrize("layout", ["bhnd", "bnhd"])
@pytest.mark.parametrize("container", ["dict", "tuple"])
def test_replay_round_trip(tmp_path, layout, container):
    B, H, N, D = 2, 3, 16, 64
    g = torch.Generator().manual_seed(0)
    qkv = [torch.randn(B, H, N, D, generator=g) for _ in range(3)]
    stored = [t.permute(0, 2, 1, 3).contiguous() if layout == "bnhd" else t for t in qkv]
    payload = dict(zip("qkv", stored)) if container == "dict" else tuple(stored)
    torch.save(payload, tmp_path / "a.pt")
    q, k, v, path = _gen("replay", shape=(B, H, N, D), dtype=torch.float16, replay_dir=tmp_path)
    assert path == tmp_path / "a.pt"
    for got, ref in zip((q, k, v), qkv):
        assert got.dtype == torch.float16 and got.is_contiguous()
        assert torch.equal(got, ref.to(torch.float16))


def test_replay_rejects_code_and_bad_shapes(tmp_path):
    torch.save({"q": torch.zeros(1), "k": torch.zeros(1)}, tmp_path / "missing.pt")
    with pytest.raises(RuntimeError, match="q, k, v"):
        _gen("replay", replay_dir=tmp_path, replay_file="missing.pt")
    torch.save({"q": torch.zeros(2, 2), "k": torch.zeros(2, 2), "v": torch.zeros(2, 2)},
               tmp_path / "shape.pt")
    with pytest.raises(RuntimeError, match="neither"):
        _gen("replay", replay_dir=tmp_path, replay_file="shape.pt")
    # an arbitrary object cannot be loaded: weights_only=True refuses it
    torch.save({"q": ValueError("x"), "k": 1, "v": 2}, tmp_path / "obj.pt")
    with pytest.raises(Exception):
        _gen("replay", replay_dir=tmp_path, replay_file="obj.pt")
    with pytest.raises(RuntimeError, match="no .pt file"):
        _gen("replay", replay_dir=tmp_path / "empty")


def test_unknown_mode():
    with pytest.raises(ValueError):
        _gen("gaussian")
