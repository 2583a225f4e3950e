"""bench.py on the CPU: the script parses, reads the committed traffic
summary for the kernels each bench line names, and refuses more than one GPU
before touching any device."""
import subprocess
import sys
from pathlib import Path

ROOT = Path(__file__).resolve().parent.parent


def test_bench_reads_committed_traffic():
    sys.path.insert(0, str(ROOT))
    import bench

    assert bench.traffic_from_profiles("plane_gemm_kernel", "c3") > 0
    assert bench.traffic_from_profiles(["pack_bt_kernel", "fused_skinny_kernel", "residue_finalize_kernel"],
                                       "gemv1") > 0
    assert bench.traffic_from_profiles(["skinny_gemm_kernel", "residue_finalize_kernel"], "gemv1_packed") > 0
    assert bench.traffic_from_profiles(["fused_native_kernel", "residue_finalize_kernel"], "c5") > 0
    assert bench.traffic_from_profiles(["plane_gemm_kernel", "residue_finalize_kernel"], "c5_packed") > 0
    assert bench.traffic_from_profiles("no_such_kernel", "c3") is None


def test_bench_refuses_several_gpus():
    r = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--gpus", "2", "--no-cpu"], capture_output=True,
                       text=True, timeout=120)
    assert r.returncode == 2
    assert "one GPU only" in r.stdout + r.stderr
