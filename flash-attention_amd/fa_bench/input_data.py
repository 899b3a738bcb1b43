"""Q, K, V generation for benchmarks and correctness runs.

Modes (the reference's benchmark/python/input_data.py:24-113 defines the
same four, and their value formulas are kept so inputs mean the same thing
in both harnesses):

  random      Q, K, V ~ N(0, 1) from a seeded generator (Q and K optionally
              scaled by qk_sigma, as config C5 does with 3).
  structured  closed-form smooth tensors of (b, h, n, d) — deterministic,
              no generator (input_data.py:33-43).
  stress      Q, K ~ 32 N(0, 1), V ~ 16 N(0, 1), plus sparse outliers
              (rate 1e-3: +256 on Q, -256 on K, +64 on V) to stress the
              online-softmax rescaling (input_data.py:46-60).
  replay      tensors from a .pt file holding dict(q, k, v) or (q, k, v),
              in [B, H, N, D] or [B, N, H, D] (permuted to BHND)
              (input_data.py:63-113).  Loaded with weights_only=True: a
              replay file can carry tensors only, never code.

Seeds: case_seed(seed, i) = seed + 100003 * i (input_data.py:11-12).
Values are drawn in float32 and rounded once to the target dtype (RNE).
"""
from __future__ import annotations

from pathlib import Path

import torch

MODES = ("random", "structured", "stress", "replay")


def case_seed(seed: int, case_index: int) -> int:
    return int(seed + case_index * 100_003)


def _gen(seed: int, device) -> torch.Generator:
    g = torch.Generator(device=device)
    g.manual_seed(seed)
    return g


def _random(shape, dtype, device, seed, qk_sigma):
    g = _gen(seed, device)
    q, k, v = (torch.randn(shape, generator=g, device=device, dtype=torch.float32)
               for _ in range(3))
    if qk_sigma != 1.0:
        q, k = q * qk_sigma, k * qk_sigma
    return q.to(dtype), k.to(dtype), v.to(dtype)


def _structured(shape, dtype, device):
    b, h, n, d = shape
    f32 = torch.float32
    bi = torch.arange(b, device=device, dtype=f32)[:, None, None, None]
    hi = torch.arange(h, device=device, dtype=f32)[None, :, None, None]
    ni = torch.arange(n, device=device, dtype=f32)[None, None, :, None]
    di = torch.arange(d, device=device, dtype=f32)[None, None, None, :]
    q = torch.sin((ni + 1) * (hi + 1) / 17.0) + 0.01 * di + 0.05 * bi
    k = torch.cos((ni + 1) * (hi + 1) / 19.0) + 0.02 * di + 0.03 * bi
    v = torch.sin((di + 1) * (hi + 1) / 23.0) + 0.001 * ni + 0.02 * bi
    return tuple(t.expand(shape).to(dtype).contiguous() for t in (q, k, v))


def _stress(shape, dtype, device, seed):
    g = _gen(seed, device)
    q = torch.randn(shape, generator=g, device=device) * 32.0
    k = torch.randn(shape, generator=g, device=device) * 32.0
    v = torch.randn(shape, generator=g, device=device) * 16.0
    rate = 1e-3
    q = q + (torch.rand(shape, generator=g, device=device) < rate).float() * 256.0
    k = k - (torch.rand(shape, generator=g, device=device) < rate).float() * 256.0
    v = v + (torch.rand(shape, generator=g, device=device) < rate).float() * 64.0
    return q.to(dtype), k.to(dtype), v.to(dtype)


def _to_bhnd(t: torch.Tensor, shape) -> torch.Tensor:
    b, h, n, d = shape
    if tuple(t.shape) == (b, h, n, d):
        return t
    if tuple(t.shape) == (b, n, h, d):
        return t.permute(0, 2, 1, 3)
    raise RuntimeError(f"replay tensor shape {tuple(t.shape)} is neither {shape} nor [B,N,H,D]")


def pick_replay_file(replay_dir, replay_file: str = "") -> Path:
    replay_dir = Path(replay_dir).expanduser()
    if replay_file:
        p = Path(replay_file).expanduser()
        if not p.is_absolute():
            p = replay_dir / p
        if not p.exists():
            raise RuntimeError(f"replay file not found: {p}")
        return p
    files = sorted(replay_dir.glob("*.pt"))
    if not files:
        raise RuntimeError(f"replay mode: no .pt file in {replay_dir}")
    return files[0]


def _replay(shape, dtype, device, replay_dir, replay_file):
    path = pick_replay_file(replay_dir, replay_file)
    obj = torch.load(path, map_location="cpu", weights_only=True)
    if isinstance(obj, dict):
        if not all(x in obj for x in ("q", "k", "v")):
            raise RuntimeError("replay dict must hold keys q, k, v")
        q, k, v = obj["q"], obj["k"], obj["v"]
    elif isinstance(obj, (list, tuple)) and len(obj) >= 3:
        q, k, v = obj[0], obj[1], obj[2]
    else:
        raise RuntimeError("replay file must hold dict(q, k, v) or a (q, k, v) sequence")
    out = tuple(_to_bhnd(t, shape).to(device=device, dtype=dtype).contiguous() for t in (q, k, v))
    return out, path


def generate_qkv(*, batch_size: int, n_heads: int, seq_len: int, d_head: int,
                 dtype: torch.dtype = torch.float16, device="cuda", input_mode: str = "random",
                 seed: int = 1234, case_index: int = 0, qk_sigma: float = 1.0,
                 replay_dir="benchmark/data/replay", replay_file: str = ""):
    """Returns (q, k, v, replay_path); replay_path is None except in replay mode."""
    shape = (batch_size, n_heads, seq_len, d_head)
    s = case_seed(seed, case_index)
    if input_mode == "random":
        q, k, v = _random(shape, dtype, device, s, qk_sigma)
        path = None
    elif input_mode == "structured":
        q, k, v = _structured(shape, dtype, device)
        path = None
    elif input_mode == "stress":
        q, k, v = _stress(shape, dtype, device, s)
        path = None
    elif input_mode == "replay":
        (q, k, v), path = _replay(shape, dtype, device, replay_dir, replay_file)
    else:
        raise ValueError(f"input_mode must be one of {MODES}, got {input_mode!r}")
    return q.contiguous(), k.contiguous(), v.contiguous(), path
