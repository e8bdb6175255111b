"""bench.py's contract pieces that need no GPU: the multi-GPU refusal, the
algorithmic work and byte counts its roofline and config-4 lines divide by,
and the traffic figure's link to the source it was measured on."""
import hashlib
import subprocess
import sys

from conftest import ROOT


def _bench():
    sys.path.insert(0, str(ROOT))
    import bench
    return bench


def test_more_than_one_gpu_exits_with_a_message():
    r = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--gpus", "2"], capture_output=True, text=True,
                       timeout=300)
    assert r.returncode == 2
    assert "one MI355X" in r.stderr and not r.stdout.strip()


def test_algorithmic_flop_per_head_chunk():
    b = _bench()
    # 2 (5 C^2 d + 3 C d^2 + C^3 / 3) for C = 64, d = 128
    assert round(b.FLOP_PER_HEAD_CHUNK) == 11_709_099
    C, d = 64, 128
    gram = 2 * C * C * d * 2          # K K^T and Q K^T
    uw = 2 * C * C * d * 2            # U = T (beta V), W = T (K scaled)
    scan = 2 * C * d * d * 3          # W S, Q S, K^T v_new
    av = 2 * C * C * d                # A v_new
    inv = 2 * C ** 3 / 3              # T = (I + L)^-1
    assert abs(b.FLOP_PER_HEAD_CHUNK - (gram + uw + scan + av + inv)) < 1


def test_config4_decode_bytes_per_token():
    b = _bench()
    assert b.model_decode_bytes() == 1_551_387_328
    # the KV rows grow with the position: 6 attention layers x 1024 halves per position
    assert b.model_decode_bytes(pos=577) - b.model_decode_bytes(pos=576) == 6 * 1024 * 2


def test_traffic_figure_is_tied_to_the_measured_source(tmp_path, monkeypatch):
    b = _bench()
    src = tmp_path / "k.hip"
    src.write_text("kernel v1\n")
    prof = tmp_path / "profiles"
    prof.mkdir()
    sha = hashlib.sha256(src.read_bytes()).hexdigest()
    (prof / "t.txt").write_text(f"# test\nsource_sha256={sha}\ntraffic_bytes=123\n")
    monkeypatch.setattr(b, "ROOT", tmp_path)
    assert b.measured_traffic("t.txt", "k.hip") == 123
    src.write_text("kernel v2\n")  # the source changed since the measurement
    assert b.measured_traffic("t.txt", "k.hip") is None
    assert b.measured_traffic("missing.txt", "k.hip") is None
