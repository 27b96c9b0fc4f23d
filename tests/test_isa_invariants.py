"""Code-generation invariants of the LDS-staged prefill GEMM (fcmoe_gemm_lds.hip).

Compiles the source to gfx950 device assembly with the library's own flags (hipcc
cross-compiles without a GPU) and checks two properties that the compiler can lose
silently and that each cost a large share of the kernel's speed when lost:

* the K loop waits on vector memory only through its own staged count(s): one
  ``s_waitcnt vmcnt(N)`` per chunk (two per pair of chunks when A stages hold two
  chunks), never ``vmcnt(0)``, which drains the prefetch ring. A second ``__shared__``
  object once made the compiler insert one per iteration (the K loop of a C4-sized
  launch went from 151 to 228 us per workgroup);
* no flat memory instructions: LDS reads typed as generic pointers become flat loads,
  which wait on vector-memory stores as well;
* the staged counts are exact: inside a K loop the only vector-memory instructions
  are the loop's own ``buffer_load ... lds`` stage loads (no scratch spill or
  reload, no other load or store), so ``vmcnt(N)`` counts exactly the loads the
  pipeline comment assigns to it; and no kernel uses scratch at all. (A spilling
  harness variant put spill/reload pairs with ``vmcnt(0)`` waits into its K loop.)
"""

from __future__ import annotations

import re
import subprocess

import pytest

from fused_cpp_amd.build import CSRC, HIP_FLAGS, ROCM

_KERNEL = re.compile(r"^(_Z\w*grouped_gemm_lds_(?:persist_)?kernel\w*):", re.M)


@pytest.fixture(scope="module")
def lds_asm(tmp_path_factory) -> str:
    hipcc = ROCM / "bin" / "hipcc"
    if not hipcc.exists():
        pytest.skip("hipcc not available")
    out = tmp_path_factory.mktemp("isa") / "fcmoe_gemm_lds.s"
    proc = subprocess.run([str(hipcc), *HIP_FLAGS, "--cuda-device-only", "-S", str(CSRC / "fcmoe_gemm_lds.hip"),
                           "-o", str(out)], capture_output=True, text=True)
    assert proc.returncode == 0, proc.stdout + proc.stderr
    return out.read_text()


def _kernels(asm: str) -> dict[str, list[str]]:
    found = {}
    for m in _KERNEL.finditer(asm):
        end = asm.index(".Lfunc_end", m.end())
        found[m.group(1)] = asm[m.end():end].splitlines()
    return found


def _k_loop(body: list[str]) -> list[str]:
    """The K loop: the smallest backward-branch region holding both MFMAs and a
    barrier (small set-up loops can be laid out with their latch after it)."""
    labels = {}
    best = None
    for i, line in enumerate(body):
        s = line.strip()
        if s.startswith(".LBB") and ":" in s:
            labels[s.split(":")[0]] = i
        elif s.startswith("s_cbranch") or s.startswith("s_branch"):
            target = s.split()[-1]
            start = labels.get(target)
            if start is None:
                continue
            region = body[start:i]
            if any("v_mfma" in x for x in region) and any("s_barrier" in x for x in region):
                if best is None or i - start < best[1] - best[0]:
                    best = (start, i)
    assert best is not None, "no K loop found"
    return body[best[0]:best[1] + 1]


def test_lds_kernels_present(lds_asm):
    names = _kernels(lds_asm)
    assert len(names) >= 12, sorted(names)


def test_k_loop_waits_on_its_own_stage_count(lds_asm):
    for name, body in _kernels(lds_asm).items():
        waits = [int(m.group(1)) for line in _k_loop(body) for m in [re.search(r"s_waitcnt vmcnt\((\d+)\)", line)] if m]
        assert 1 <= len(waits) <= 2, (name, waits)
        assert all(w > 0 for w in waits), (name, waits)


def test_no_flat_memory_instructions(lds_asm):
    for name, body in _kernels(lds_asm).items():
        flat = [line.strip() for line in body if line.strip().startswith("flat_")]
        assert not flat, (name, flat[:3])


_VMEM = ("buffer_", "global_", "scratch_", "flat_")


def test_k_loop_vector_memory_is_only_its_stage_loads(lds_asm):
    for name, body in _kernels(lds_asm).items():
        ops = [line.strip() for line in _k_loop(body) if line.strip().startswith(_VMEM)]
        assert ops, name
        other = [op for op in ops if not (op.startswith("buffer_load_dwordx4") and op.split(";")[0].rstrip().endswith("lds"))]
        assert not other, (name, other[:3])


def test_no_kernel_uses_scratch(lds_asm):
    sizes = [int(v) for v in re.findall(r"\.private_segment_fixed_size:\s+(\d+)", lds_asm)]
    assert sizes and all(v == 0 for v in sizes), sizes


def _vgprs(asm: str) -> dict[str, int]:
    """VGPR count of every kernel in a device assembly file (from its metadata)."""
    names = re.findall(r"^\s+\.name:\s+(\S+)", asm, re.M)
    counts = [int(v) for v in re.findall(r"^\s+\.vgpr_count:\s+(\d+)", asm, re.M)]
    assert len(names) == len(counts), (len(names), len(counts))
    return dict(zip(names, counts))


def test_mixed_plan_register_budget(lds_asm, tmp_path):
    """The mixed prefill plan relies on one workgroup of the persistent MFMA
    kernel (two waves per SIMD) and one of the 16-row streaming kernel (one
    wave per SIMD) sharing every CU: 2 x 216 + 80 <= 512 VGPRs (allocation
    granule 8). A kernel that grows past its budget silently loses the
    co-residency (C3 2.9 -> 5.6 ms when the MFMA kernel reached 225)."""
    hipcc = ROCM / "bin" / "hipcc"
    out = tmp_path / "fcmoe_gemm.s"
    proc = subprocess.run([str(hipcc), *HIP_FLAGS, "--cuda-device-only", "-S", str(CSRC / "fcmoe_gemm.hip"),
                           "-o", str(out)], capture_output=True, text=True)
    assert proc.returncode == 0, proc.stdout + proc.stderr
    mfma = {k: v for k, v in _vgprs(lds_asm).items() if "grouped_gemm_lds_persist_kernelILb1E" in k}
    stream = {k: v for k, v in _vgprs(out.read_text()).items() if "grouped_gemm_stream_kernelILb1E" in k}
    assert mfma and stream
    rnd = lambda v: (v + 7) // 8 * 8  # noqa: E731
    assert all(rnd(v) <= 216 for v in mfma.values()), mfma
    assert all(rnd(v) <= 80 for v in stream.values()), stream
    assert 2 * max(rnd(v) for v in mfma.values()) + max(rnd(v) for v in stream.values()) <= 512
