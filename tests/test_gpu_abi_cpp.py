"""The C ABI from a C++ caller: tests/abi/iek_abi_test.cpp and the bench_compare CLI
(inference_engine_rust_amd/cli/bench_compare.cpp), both built with g++ against the static libiek.a
by the package build. The GPU tests drive load -> prefill -> greedy generation through
include/iek.h and compare the tokens with the golden C0 run; the CPU tests check the CLI's
argument handling, which fails before any device call.
"""
import json
import os
import subprocess

import pytest

from inference_engine_rust_amd import build as B

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")
ABI_TEST = os.path.join(B.BIN, "iek_abi_test")
BENCH = os.path.join(B.BIN, "iek_bench_compare")


def _run(cmd, timeout=180):
    return subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.PIPE, text=True, timeout=timeout)


def test_tools_are_built():
    assert os.access(ABI_TEST, os.X_OK) and os.access(BENCH, os.X_OK)
    assert os.path.exists(B.LIB_A)


def test_bench_compare_rejects_fewer_than_five_runs():
    r = _run([BENCH, "--runs", "3", "all"])
    assert r.returncode == 6 and "--runs must be at least 5" in r.stderr  # EngineError::Model


def test_bench_compare_needs_a_suite():
    r = _run([BENCH, "--json"])
    assert r.returncode == 2 and "subcommand" in r.stderr


@pytest.mark.gpu
def test_cpp_caller_load_prefill_generate(gpu, c0_path):
    g = json.load(open(os.path.join(GOLDEN, "c0_seed0.json")))
    r = _run([ABI_TEST, c0_path, str(g["n_decode"]), *[str(t) for t in g["prompt"]]])
    assert r.returncode == 0, r.stderr
    out = json.loads(r.stdout.strip().splitlines()[-1])
    assert out["tokens"] == g["tokens"]
    assert out["checks"] > 20


@pytest.mark.gpu
def test_bench_compare_all_suites(gpu, c0_path):
    r = _run([BENCH, "--model", c0_path, "--prompt-tokens", "16", "--runs", "5", "--json", "all",
              "--decode-tokens", "8"])
    assert r.returncode == 0, r.stderr
    out = json.loads(r.stdout)
    assert out["suite"] == "all" and len(out["prompt_ids"]) == 16
    assert len(out["runs"]["cold"]) == len(out["runs"]["interactive"]) == len(out["runs"]["decode"]) == 5
    for c in out["runs"]["cold"]:
        assert c["cold_ttft_ms"] >= c["prompt_eval_ms"] + c["lm_head_sample_ms"] > 0
        assert c["tensor_load_ms"] > 0
    for m in out["runs"]["interactive"]:
        assert abs(m["ttft_infer_ms"] - (m["prefill_prepare_ms"] + m["prompt_eval_ms"] + m["lm_head_sample_ms"])) < 1e-3
    d = out["summary"]["decode"]["decode_tokens_per_sec"]
    assert d["min"] <= d["median"] <= d["max"] and d["min"] <= d["p95"] <= d["max"]
    # the throughput gate fails the run (EngineError::Model)
    r = _run([BENCH, "--model", c0_path, "--prompt-tokens", "8", "--runs", "5", "--min-decode-tps", "1e12",
              "decode-throughput", "-n", "4"])
    assert r.returncode == 6 and "min-decode-tps" in r.stderr
