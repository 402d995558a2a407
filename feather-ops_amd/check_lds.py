#!/usr/bin/env python3
"""Check every kernel instantiation's real LDS allocation against the size its tile asks for.

The number the runtime allocates is the code object's `group_segment_fixed_size`; the kernels ask for a
compile-time function of the tile (the ring kernel: its activation and weight rings, `tiles.ring_slots`,
shallow or deep; the wide kernel: its 3 + 3 slots of 256 x 64 activation and 256 or 192 x 64 weight stages;
the streaming kernel: per-wave activation double buffers plus the K-slice join). A mismatch costs
occupancy, so it is a bug in the source or the compiler. Same role as the reference's
`tools/check_lds.py:30-101`, for gfx950: it compiles `csrc/scaled_mm_launch.hip` for one dtype
combination to assembly (device code only, ~10 s) and reads `.amdhsa_group_segment_fixed_size` per kernel.

    python check_lds.py                 # e5m2 weights, fp16 activations, fp16 output
    python check_lds.py --combo 011     # <e5m2><a_bf16><out_bf16>
"""

import argparse
import importlib.util
import pathlib
import re
import subprocess
import sys

HERE = pathlib.Path(__file__).resolve().parent
ROOT = HERE.parent
HIPCC = "/opt/rocm/bin/hipcc"


def _tiles():
    spec = importlib.util.spec_from_file_location("_feather_tiles", HERE / "feather_ops" / "tiles.py")
    module = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(module)
    return module


def expected_bytes(kernel: str, ints: list[int], bools: list[int] = ()) -> int:
    """LDS bytes the kernel's tile asks for (the kernels' `kLdsBytes`); a ring kernel's fifth template
    flag is its deep-ring variant (the flags after it, such as non-temporal weight loads, leave LDS alone)."""
    if kernel == "wide_kernel":
        repeat_n = ints[0]
        slots_a, slots_b = _tiles().ring_slots((2, 2, 4, 8, repeat_n, 1))
        return slots_a * 256 * 64 * 2 + slots_b * 32 * repeat_n * 64
    if kernel == "ring_dma_kernel":
        warps_m, warps_n, unroll_k, repeat_m, repeat_n = ints
        deep = bool(bools[4]) if len(bools) >= 5 else False
        slots_a, slots_b = _tiles().ring_slots((warps_m, warps_n, unroll_k, repeat_m, repeat_n, 1), deep)
        a_stage = 16 * warps_m * repeat_m * unroll_k * 32
        b_stage = 16 * warps_n * repeat_n * unroll_k * 16
        return slots_a * a_stage + slots_b * b_stage
    k_slices, warps_n, unroll_k, repeat_m, repeat_n = ints
    # fetches in flight per wave (StreamShape::kDepth)
    depth = 3 if k_slices * warps_n * repeat_n * (unroll_k // 4) <= 8 and repeat_m <= 2 else 2
    activations = k_slices * warps_n * depth * (unroll_k // 4) * repeat_m * 2048
    join = (k_slices if k_slices > 1 else 0) * warps_n * repeat_m * repeat_n * 64 * 16
    return activations + join


def compile_asm(combo: str) -> str:
    e5m2, a_bf16, out_bf16 = combo
    command = [
        HIPCC, "--offload-arch=gfx950", "-O3", "-std=c++17", "-Wno-unused-command-line-argument",
        "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
        f"-I{HERE / 'csrc'}", f"-I{ROOT / 'include'}",
        f"-DFEATHER_B_E5M2={e5m2}", f"-DFEATHER_A_BF16={a_bf16}", f"-DFEATHER_OUT_BF16={out_bf16}",
        "--offload-device-only", "-S", "-o", "-", str(HERE / "csrc" / "scaled_mm_launch.hip"),
    ]
    result = subprocess.run(command, capture_output=True, text=True, check=False)
    if result.returncode != 0:
        raise SystemExit(f"compiling {combo} for gfx950 exited with {result.returncode}; end of its stderr:\n"
                         f"{result.stderr[-4000:]}")
    return result.stdout


def audit(asm: str) -> tuple[int, list[tuple]]:
    """(instantiations checked, [(kernel, ints, bools, allocated, expected)] that disagree)."""
    # A kernel's mangled name carries its template arguments as `L<type><value>E` tokens after `I`: `i` for
    # the int tile parameters, `b` for the bool flags.
    kernel_re = re.compile(r"(ring_dma_kernel|stream_kernel|wide_kernel)I(.*)")
    name, checked, bad = None, 0, []
    for line in asm.splitlines():
        kd = re.match(r"\s*\.amdhsa_kernel\s+(\S+)", line)
        if kd:
            name = kd.group(1)
            continue
        if name is None or ".amdhsa_group_segment_fixed_size" not in line:
            continue
        match = kernel_re.search(name)
        name = None
        if not match:
            continue
        tokens = re.findall(r"L([ib])(\d+)E", match.group(2))
        ints = [int(v) for kind, v in tokens if kind == "i"]
        bools = [int(v) for kind, v in tokens if kind == "b"]
        allocated = int(line.split()[-1])
        expected = expected_bytes(match.group(1), ints, bools)
        checked += 1
        if allocated != expected:
            bad.append((match.group(1), tuple(ints), tuple(bools), allocated, expected))
    return checked, bad


def main() -> int:
    parser = argparse.ArgumentParser()
    parser.add_argument("--combo", default="100", choices=[f"{i:03b}" for i in range(8)],
                        help="<e5m2><a_bf16><out_bf16>")
    args = parser.parse_args()
    checked, bad = audit(compile_asm(args.combo))
    print(f"{checked} kernel instantiations checked against their tile's LDS size")
    if checked == 0:
        print("no kernel metadata found")
        return 1
    if not bad:
        print("each instantiation allocates exactly its tile's LDS")
        return 0
    print(f"{len(bad)} mismatches (kernel, ints, bools, allocated, expected):")
    for entry in bad:
        print(" ", *entry)
    return 1


if __name__ == "__main__":
    sys.exit(main())
