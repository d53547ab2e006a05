"""CPU checks of bench.py's contract that need no GPU: the one-GPU guard and the
algorithmic byte counts its roofline uses."""
import subprocess
import sys
from pathlib import Path

ROOT = Path(__file__).resolve().parent.parent


def test_more_than_one_gpu_is_refused():
    r = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--gpus", "2"], capture_output=True, text=True,
                       timeout=120)
    assert r.returncode == 2
    assert "one GPU" in r.stderr
    assert r.stdout == ""


def test_algorithmic_bytes():
    sys.path.insert(0, str(ROOT))
    import bench
    # tiles I*O*K/8 + fp16 suh [I] + fp16 svh [O]
    assert bench.matrix_bytes(2048, 512, 8) == 2048 * 512 * 4 // 8 + 2 * 2048 + 2 * 512
    # one config-3 expert at 4 bpw: gate + up (2048 -> 512) and down (512 -> 2048)
    assert bench.expert_bytes(8, 8) == 1_588_224
