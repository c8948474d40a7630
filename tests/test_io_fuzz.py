"""Mutation fuzz of the C++ snapshot readers under AddressSanitizer / UBSan (CPU).

tests/host_cpp/fuzz_io.cpp mutates the golden safetensors fixture's JSON header and a config.json
(byte overwrites, inserted JSON tokens, erasures, truncation, inconsistent header lengths) and
feeds each case to mlxq::read_safetensors / mlxq::write_quantized_config
(mlx-gen_amd/host/io.cpp).  Every case must parse into tensors whose bytes match their shapes or
raise mlxq::Error; a sanitizer report aborts the program and fails the test.
"""
import os
import subprocess

import pytest

HERE = os.path.dirname(__file__)
EXE = os.path.join(HERE, "host_cpp", "fuzz_io")
FIXTURE = os.path.join(HERE, "golden", "quant_q4q8.safetensors")


@pytest.mark.parametrize("seed", [1, 2])
def test_snapshot_reader_fuzz(tmp_path, seed):
    assert os.path.exists(EXE), "build() compiles tests/host_cpp/fuzz_io"
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=0:abort_on_error=1",
               UBSAN_OPTIONS="print_stacktrace=1:halt_on_error=1")
    r = subprocess.run([EXE, FIXTURE, str(tmp_path), str(seed), "1500"], env=env, capture_output=True,
                       text=True, timeout=300)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "1500 cases" in r.stdout
    # the mutations reach both outcomes: some files still parse, most are refused
    parsed = int(r.stdout.split(" parsed")[0].split(", ")[-1])
    assert 0 < parsed < 1500, r.stdout
