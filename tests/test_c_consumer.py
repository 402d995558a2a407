"""The C ABI from a compiled, torch-free consumer (tests/c_abi/feather_consumer.c), as the reference's
cpp_benchmarks/benchmark_scaled_mm_hip.cpp:27-47,150-290 binds `launch_scaled_mm`: the header is compiled
by gcc and linked against libfeather_ops_gfx950.so, so a declaration that drifts from the library breaks
the build. CPU: the contract refusals. GPU: prepack + launch + split-K launch on hipMalloc'd buffers
against the oracle.
"""

import pathlib
import subprocess

import numpy as np
import pytest
import torch

from gpu_helpers import check_against_oracle
from oracle import naive as oracle

HERE = pathlib.Path(__file__).resolve().parent
SRC = HERE / "c_abi"
BUILT = SRC / "_build" / "feather_consumer"


def test_header_compiles_links_and_refuses_out_of_contract_calls(tmp_path):
    """A fresh gcc build of the consumer against include/feather_ops.h, then its host-only refusal checks
    (every out-of-contract call returns false before any GPU work)."""
    import os

    subprocess.run(["make", "-C", str(SRC), "-B", f"OUT={tmp_path}"], check=True, capture_output=True)
    lib_dir = HERE.parent / "feather-ops_amd" / "feather_ops"  # the build's rpath is relative to tests/c_abi/_build
    env = {**os.environ, "LD_LIBRARY_PATH": f"{lib_dir}:{os.environ.get('LD_LIBRARY_PATH', '')}"}
    done = subprocess.run([str(tmp_path / "feather_consumer"), "refuse"], capture_output=True, text=True,
                          timeout=120, env=env)
    assert done.returncode == 0, done.stderr
    assert "refusals ok" in done.stdout


@pytest.mark.gpu
@pytest.mark.parametrize("m,n,k,a_fmt,tile,splits", [
    (300, 1000, 1040, oracle.BF16, (2, 2, 4, 4, 4, 1), 2),     # ring kernel, ragged M and N, split 2 ways
    (16, 4096, 4096, oracle.F16, (8, 1, 4, 1, 4, 0), 3),       # streaming kernel, split 3 ways
])
def test_consumer_runs_on_the_gpu(tmp_path, m, n, k, a_fmt, tile, splits):
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    assert BUILT.exists(), "build tests/c_abi first (make -C tests/c_abi, run by __graft_entry__.build())"
    a_bits, packed, scale, b_codes = oracle.make_inputs(m, k, n, a_fmt, seed=4)
    out_fmt = a_fmt
    out_dt = torch.bfloat16 if out_fmt == oracle.BF16 else torch.float16
    bias = torch.randn(n, generator=torch.Generator().manual_seed(5)).to(out_dt)
    bias_bits = bias.view(torch.int16).numpy().view(np.uint16)
    a_bits.tofile(tmp_path / "a.bin")
    b_codes.tofile(tmp_path / "b.bin")
    np.array([scale], np.float32).tofile(tmp_path / "scale.bin")
    bias_bits.tofile(tmp_path / "bias.bin")
    args = [str(BUILT), "run", str(tmp_path), str(m), str(n), str(k), str(int(a_fmt == oracle.BF16)),
            str(int(out_fmt == oracle.BF16)), *[str(int(v)) for v in tile], str(splits)]
    print("consumer:", " ".join(args[1:]), flush=True)
    done = subprocess.run(args, capture_output=True, text=True, timeout=120)
    assert done.returncode == 0, done.stderr
    print(done.stdout.strip())

    a_dt = torch.bfloat16 if a_fmt == oracle.BF16 else torch.float16
    a = torch.from_numpy(a_bits.view(np.int16)).view(a_dt)
    bp = torch.from_numpy(packed).view(torch.float8_e5m2)
    s = torch.tensor(scale, dtype=torch.float32)
    for name in ("c.bin", "c_split.bin"):
        c_bits = np.fromfile(tmp_path / name, dtype=np.uint16).reshape(m, n)
        out = torch.from_numpy(c_bits.view(np.int16)).view(out_dt)
        check_against_oracle(out, a, bp, s, bias)
    if a_fmt == oracle.BF16:  # widened once from C, then the fp16-activation launch: the in-place bits
        assert np.array_equal(np.fromfile(tmp_path / "c_widened.bin", dtype=np.uint16),
                              np.fromfile(tmp_path / "c.bin", dtype=np.uint16))
