"""Build properties of the gfx950 forward kernels, read from the device
assembly that hipcc emits for csrc/fa_fwd_kernel.hip with the library's own
flags (CPU only: hipcc cross-compiles without a GPU).

- Every forward variant fits two waves per SIMD (at most 256 VGPRs, no
  AGPRs), with no scratch and no VGPR spills; the pair-mode variants hold two
  K/V rings (128 KiB at D = 128, one workgroup per CU).
- m0 discipline of the K/V staging: the DMA is issued from inline asm that
  sets m0 (the LDS destination) immediately before each
  global_load_lds_dwordx4 and declares m0 clobbered.  The compiler does not
  save a reserved register around such an asm, so the kernels must not use
  m0 for anything else: every m0 reference in the assembly is one of those
  writes, and each is followed by its DMA instruction.
"""
from __future__ import annotations

import os
import re
import shutil
import subprocess
import sys

import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, os.path.join(REPO, "flash-attention_amd"))


@pytest.fixture(scope="module")
def device_asm(tmp_path_factory):
    import build as fa_build  # flash-attention_amd/build.py

    try:
        hipcc = fa_build._hipcc()
    except RuntimeError:
        pytest.skip("hipcc not available")
    out = str(tmp_path_factory.mktemp("asm") / "fa_fwd_kernel.s")
    flags = [f for f in fa_build.HIP_FLAGS if f not in ("-fPIC", "-Wall")]
    cmd = [hipcc, *flags, "-I", fa_build.INCLUDE, "-I", fa_build.CSRC, "-x", "hip",
           "--cuda-device-only", "-S", os.path.join(fa_build.CSRC, "fa_fwd_kernel.hip"),
           "-o", out]
    proc = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    assert proc.returncode == 0, proc.stdout[-4000:]
    with open(out) as f:
        return f.read()


def _kernel_metadata(asm: str):
    """(name, {field: value}) per kernel from the amdhsa.kernels metadata."""
    meta = asm[asm.index("amdhsa.kernels:"):]
    kernels = []
    for block in re.split(r"\n  - ", meta)[1:]:
        fields = dict(re.findall(r"^    \.(\w+):\s+(\S+)$", block, re.M))
        if "name" in fields:
            kernels.append((fields["name"], fields))
    return kernels


def test_forward_variants_fit_two_waves_per_simd(device_asm):
    kernels = _kernel_metadata(device_asm)
    fwd = [(n, f) for n, f in kernels if "fa_fwd_kernel" in n]
    # template arguments <D, BF16, CAUSAL, NW, SPLIT, PAIR, LSE_L>
    args = {n: re.search(r"fa_fwd_kernelILi(\d+)ELb(\d)ELb(\d)ELi(\d)ELb(\d)ELb(\d)ELb(\d)E", n).groups()
            for n, _ in fwd}
    pair = [n for n, a in args.items() if a[5] == "1"]
    assert len(fwd) == 46, [n for n, _ in kernels]
    # pair mode: causal, 8 waves, unsplit, D 64/128 x fp16/bf16 (bf16 also
    # in its LSE_L form)
    assert len(pair) == 6 and all(args[n][2] == "1" and args[n][3] == "8" and args[n][4] == "0"
                                  for n in pair)
    # LSE_L: only bf16 kernels with an optimistic pass (pair mode, split chunks)
    lse_l = [a for a in args.values() if a[6] == "1"]
    assert len(lse_l) == 10 and all(a[1] == "1" and (a[4] == "1" or a[5] == "1") for a in lse_l)
    assert sum("fa_merge_kernel" in n for n, _ in kernels) == 4
    # the 16x16x32 kernels <D, BF16, CAUSAL, NW, LSE_L>, D = 64 and 128: fp16
    # and bf16, causal and non-causal, with 4 and 8 waves (no fp16 non-causal
    # 4-wave one at D = 64, which runs the 32x32x16 kernel); bf16 in two
    # forms (with and without the LSE's unrounded sums in the optimistic
    # pass), fp16 in one
    k16 = {re.search(r"fa_fwd16_kernelILi(\d+)ELb(\d)ELb(\d)ELi(\d)ELb(\d)E", n).groups(): f
           for n, f in kernels if "fa_fwd16_kernel" in n}
    assert len(k16) == 23 and {k[0] for k in k16} == {"64", "128"}, sorted(k16)
    assert sum(k[0] == "128" for k in k16) == 12, sorted(k16)
    assert not any(k[0] == "64" and k[1:4] == ("0", "0", "4") for k in k16), sorted(k16)
    assert not any(k[1] == "0" and k[4] == "1" for k in k16), sorted(k16)
    for (d, bf16, causal, nw, lse_l), f in k16.items():
        # the same 4-tile K/V ring, plus the optimistic pass's flag where it runs
        ring = 4 * 64 * 2 * int(d)
        opt = bf16 == "1" or causal == "0" or nw == "8"
        assert int(f["group_segment_fixed_size"]) == ring + (4 if opt else 0), (d, bf16, causal, nw)
    for name, f in kernels:
        assert int(f["private_segment_fixed_size"]) == 0, (name, "scratch")
        assert int(f["vgpr_spill_count"]) == 0, (name, "VGPR spills")
        assert int(f.get("agpr_count", "0")) == 0, (name, "AGPRs")
        assert int(f["vgpr_count"]) <= 256, (name, f["vgpr_count"])
    for name, f in fwd:
        # K/V ring: 4 tiles of 64 keys x D fp16, two such rings in pair mode
        # (+ the optimistic pass's flag).
        d = 128 if "Li128E" in name else 64
        ring = (8 if name in pair else 4) * 64 * 2 * d
        assert int(f["group_segment_fixed_size"]) in (ring, ring + 4), name


def test_m0_only_set_for_the_staging_dma(device_asm):
    lines = [ln.strip() for ln in device_asm.splitlines()]
    code = [ln for ln in lines if ln and not ln.startswith(";") and not ln.startswith(".")]
    m0_refs = [i for i, ln in enumerate(code) if re.search(r"\bm0\b", ln)]
    dma = [i for i, ln in enumerate(code) if ln.startswith("global_load_lds_dwordx4")]
    assert dma, "no staging DMA found"
    assert len(m0_refs) == len(dma)
    for i in m0_refs:
        assert re.fullmatch(r"s_mov_b32 m0, s\d+", code[i]), code[i]
        assert code[i + 1].startswith("global_load_lds_dwordx4"), (code[i], code[i + 1])
