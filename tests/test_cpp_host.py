"""Runs the C++ tests of the host layer (tests/cpp): the mirrored mensurflow API -- Tensor,
Dispatcher, Registry and the ops -- with the CPU side served by the oracle and, under -m gpu,
the rocm device served by the HIP kernels through the C ABI."""
import os
import subprocess

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
CPP = os.path.join(HERE, "cpp")
TESTS = ["core_test", "blas_test", "attention_test", "tuning_test", "reference_cases_test"]


def binary(name):
    path = os.path.join(CPP, "bin", name)
    if not os.path.exists(path):
        subprocess.run(["make", "-s", "-C", CPP], check=True)
    return path


def run(name, *flags, timeout=600):
    proc = subprocess.run([binary(name), *flags], capture_output=True, text=True, timeout=timeout)
    out = proc.stdout + proc.stderr
    print(out)
    assert proc.returncode == 0, out
    assert f"{name} passed" in out


@pytest.mark.parametrize("name", TESTS)
def test_host_layer_cpu(name):
    run(name, "--cpu-only")


@pytest.mark.gpu
@pytest.mark.parametrize("name", TESTS)
def test_host_layer_rocm(name):
    run(name, "--require-gpu")


def test_device_gelu_arithmetic_every_61st_float():
    """The device's tanh gelu (csrc/gelu_tanh.hpp, the same operations compiled for the CPU)
    gives the oracle's bits on every 61st float bit pattern (70 M inputs) for three stand-ins of
    the reciprocal instruction. `gelu_exhaustive_test --stride 1` covers all 2^32 (about 90 s on
    8 threads; it passes as well)."""
    run("gelu_exhaustive_test", "--stride", "61")
