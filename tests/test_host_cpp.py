"""The C++ host drivers without a GPU: command-line contract and the
argument errors of run_deltanet_chunk_rule (deltanet_chunk.cpp:53-75 messages),
which are raised before any device call."""
import subprocess

import numpy as np
import pytest

import host_cli as H
from spock_amd import synth


def _small(H_=2, T=5, dk=3, dv=2):
    inp = synth.chunk_inputs(H_, T, dk=dk, dv=dv, seed=3, l2=False)
    return H.chunk_fixture(inp["q"], inp["k"], inp["v"], inp["g"], inp["beta"])


@pytest.fixture(scope="module", autouse=True)
def _built():
    if not (H.CHUNK_CLI.exists() and H.SESSION_CLI.exists()):
        pytest.fail("C++ drivers are not built (python -c 'import __graft_entry__ as g; g.build()')")


def test_chunk_cli_usage():
    r = subprocess.run([str(H.CHUNK_CLI)], capture_output=True, text=True)
    assert r.returncode == 2 and "--input is required" in r.stderr
    # as in the reference driver (apps/spock-deltanet-chunk.cpp:42-50): a
    # trailing --input without a FILE counts as no input, other arguments are
    # ignored
    r = subprocess.run([str(H.CHUNK_CLI), "--input"], capture_output=True, text=True)
    assert r.returncode == 2 and "--input is required" in r.stderr
    r = subprocess.run([str(H.CHUNK_CLI), "--bogus"], capture_output=True, text=True)
    assert r.returncode == 2 and "--input is required" in r.stderr
    r = subprocess.run([str(H.CHUNK_CLI), "--bogus", "--input", "/nonexistent/request.json", "-x"],
                       capture_output=True, text=True)
    assert r.returncode == 1 and "/nonexistent/request.json" in r.stderr
    r = subprocess.run([str(H.CHUNK_CLI), "--help"], capture_output=True, text=True)
    assert r.returncode == 0 and r.stdout.startswith("usage: spock-deltanet-chunk")


@pytest.mark.parametrize("field,expect", [
    ("query", "query size mismatch: expected 30, got 29"),
    ("key", "key size mismatch: expected 30, got 29"),
    ("value", "value size mismatch: expected 20, got 19"),
    ("g", "g size mismatch: expected 10, got 9"),
    ("beta", "beta size mismatch: expected 10, got 9"),
])
def test_chunk_size_mismatch(tmp_path, field, expect):
    fx = _small()
    fx[field] = fx[field][:-1]
    r = H.run_chunk_cli(tmp_path, fx)
    assert r.returncode == 1 and r.stderr.strip() == f"spock-deltanet-chunk: {expect}"


def test_chunk_initial_state_mismatch(tmp_path):
    fx = _small()
    fx["initial_state"] = [0.0] * 11
    r = H.run_chunk_cli(tmp_path, fx)
    assert r.returncode == 1 and "initial_state size mismatch: expected 12, got 11" in r.stderr


@pytest.mark.parametrize("field", ["num_heads", "sequence_length", "key_dim", "value_dim", "chunk_size"])
def test_chunk_zero_config_field(tmp_path, field):
    fx = _small()
    fx[field] = 0
    r = H.run_chunk_cli(tmp_path, fx)
    assert r.returncode == 1 and "DeltaNet chunk config fields must be non-zero" in r.stderr


def test_chunk_json_errors(tmp_path):
    r = H.run_chunk_cli(tmp_path, '{"num_heads": 2, ')
    assert r.returncode == 1 and "JSON parse error" in r.stderr
    r = H.run_chunk_cli(tmp_path, "[1, 2]")
    assert r.returncode == 1 and "top-level JSON value is not an object" in r.stderr
    cases = [
        ("use_qk_l2norm", 1, 'field "use_qk_l2norm": expected true or false'),
        ("beta", None, 'field "beta": required array of numbers is missing'),
        ("query", {"a": 1}, 'field "query": expected an array of numbers'),
        ("num_heads", None, 'field "num_heads": required integer is missing'),
        ("key_dim", 2.5, 'field "key_dim": expected a non-negative integer'),
        ("value_dim", -1, 'field "value_dim": expected a non-negative integer'),
        ("chunk_size", "64", 'field "chunk_size": expected an integer'),
    ]
    for field, value, msg in cases:
        fx = _small()
        if value is None:
            del fx[field]
        else:
            fx[field] = value
        r = H.run_chunk_cli(tmp_path, fx)
        assert r.returncode == 1 and msg in r.stderr, (field, r.stderr)
    fx = _small()
    fx["g"][3] = "x"
    r = H.run_chunk_cli(tmp_path, fx)
    assert r.returncode == 1 and 'field "g": element 3 is not a number' in r.stderr


def test_chunk_head_width_limit(tmp_path):
    inp = synth.chunk_inputs(1, 2, dk=129, dv=4, seed=1, l2=False)
    r = H.run_chunk_cli(tmp_path, H.chunk_fixture(inp["q"], inp["k"], inp["v"], inp["g"], inp["beta"]))
    assert r.returncode == 1 and "key_dim and value_dim must be at most 128" in r.stderr


def test_session_cli_usage(tmp_path):
    r = subprocess.run([str(H.SESSION_CLI)], capture_output=True, text=True)
    assert r.returncode == 2 and "--input and --output are required" in r.stderr
    r = subprocess.run([str(H.SESSION_CLI), "--input", str(tmp_path), "--output", str(tmp_path)],
                       capture_output=True, text=True)
    assert r.returncode == 1 and "cannot open" in r.stderr and "meta.json" in r.stderr
