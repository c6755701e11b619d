"""The launch planners' LDS arithmetic (blog_amd/csrc/qlin_plan.hpp), on the CPU: tests/plan_check.cpp
is built with g++ against the same header the kernels' launchers include, and run."""
import os
import subprocess

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_planners_fit_lds_up_to_the_edge(tmp_path):
    exe = tmp_path / "plan_check"
    subprocess.run(["g++", "-std=c++17", "-O1", "-Wall", "-Werror", f"-I{os.path.join(ROOT, 'blog_amd', 'csrc')}",
                    os.path.join(ROOT, "tests", "plan_check.cpp"), "-o", str(exe)], check=True)
    r = subprocess.run([str(exe)], capture_output=True, text=True)
    assert r.returncode == 0, r.stdout + r.stderr
    assert r.stdout.startswith("ok")
