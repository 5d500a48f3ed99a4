"""The C API driven by a program compiled as C (tests/c/run_certex_c.c), as the reference's
c/tests/neighbors/run_certex_c.c + certex_c.cu do: build from a host dataset, search with and
without a bitset, remove, reject mismatched query types; every id and distance checked against a
brute force inside the program."""

import os
import subprocess

import pytest

pytestmark = pytest.mark.gpu
HERE = os.path.dirname(os.path.abspath(__file__))
EXE = os.path.join(HERE, "c", "_build", "run_certex_c")


def test_c_program(gpu):
    if not os.path.exists(EXE):
        subprocess.run(["make", "-s", "-C", os.path.join(HERE, "c")], check=True)
    r = subprocess.run([EXE], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "run_certex_c: ok" in r.stdout
