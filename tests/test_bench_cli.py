"""bench.py's command-line contract on the CPU: more than one GPU is refused with a message
(bench.py measures one GPU), and every workload name is accepted by the parser."""
import subprocess
import sys
from pathlib import Path

ROOT = Path(__file__).resolve().parents[1]


def test_more_than_one_gpu_is_refused_with_a_message():
    r = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--gpus", "2"], capture_output=True, text=True,
                       timeout=120, cwd=ROOT)
    assert r.returncode == 2
    assert "one GPU" in r.stderr and not r.stdout.strip()


def test_help_lists_every_workload():
    r = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--help"], capture_output=True, text=True,
                       timeout=120, cwd=ROOT)
    assert r.returncode == 0
    for w in ("qwen25_3b_b64", "llama31_8b_b128", "qwen25_3b_prefill", "qwen25_3b_step36",
              "qwen25_3b_sampling", "qwen25_3b_rope_append"):
        assert w in r.stdout
