"""The C++ host API (libmla_host.so, cpp_inference_train_engine_amd/host/mla_host.hpp)
through its own C++ tests (tests/host/test_host.cpp, built by tests/host/Makefile):
the sampler's and tokenizer's known answers on the host, and on the GPU a HipExecution
against the CPU decoder (the reference's test_mps.cpp:126-166 pattern), forks and input
errors, InferenceEngine on a model export, and the batched Server."""
import os
import subprocess

import numpy as np
import pytest

from conftest import GOLDEN, REPO, TINY

BIN = os.path.join(REPO, "tests", "host", "test_host")
HOST_LIB = os.path.join(REPO, "cpp_inference_train_engine_amd", "libmla_host.so")


def _run(args, timeout):
    res = subprocess.run([BIN, *args], capture_output=True, text=True, timeout=timeout)
    print(res.stdout + res.stderr, flush=True)
    return res


def test_host_library_exports_the_interfaces():
    assert os.path.exists(HOST_LIB) and os.path.exists(BIN), "run __graft_entry__.build() first"
    names = subprocess.run(["nm", "-DC", "--defined-only", HOST_LIB], capture_output=True,
                           text=True, check=True).stdout
    for sym in ("mla_host::HipEngine::create", "mla_host::HipEngine::load",
                "mla_host::make_hip_execution", "mla_host::Tokenizer::load",
                "mla_host::InferenceEngine::load", "mla_host::InferenceEngine::generate_tokens",
                "mla_host::sample_token", "mla_host::Server::create", "mla_host::Server::poll"):
        assert sym in names, sym


def test_host_api_cpu_tests():
    res = _run(["--cpu", GOLDEN], 120)
    assert res.returncode == 0 and "0 failed checks" in res.stdout


@pytest.mark.gpu
def test_host_api_gpu_tests(gpu, tiny_fixture, tmp_path):
    from oracle.export_format import write_export
    with open(os.path.join(GOLDEN, "tokenizer_tiny.json"), "rb") as f:
        tok = f.read()
    export = str(tmp_path / "model")
    write_export(export, TINY, np.asarray(tiny_fixture["params"], np.float32), tok, "f16")
    res = _run(["--gpu", GOLDEN, export], 180)
    assert res.returncode == 0 and "0 failed checks" in res.stdout
    assert res.stdout.count("PASS ") == 9
