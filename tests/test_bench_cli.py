"""bench.py's command-line contract, on the CPU (no GPU is touched): more
than one GPU is refused with a JSON error line and exit status 2 (this build
measures one GPU), the two-stream probe is refused outside the hero GEMV and
the read floor, and every workload names a kind that main() dispatches."""
import ast
import json
import os
import subprocess
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
BENCH = os.path.join(ROOT, "bench.py")


def _run(*args):
    env = dict(os.environ, HIP_VISIBLE_DEVICES="")
    p = subprocess.run([sys.executable, BENCH, *args], capture_output=True, text=True, timeout=300, cwd=ROOT, env=env)
    lines = [ln for ln in p.stdout.splitlines() if ln.strip()]
    return p.returncode, json.loads(lines[-1]) if lines else None


def test_more_than_one_gpu_is_refused():
    rc, rec = _run("--gpus", "2")
    assert rc == 2
    assert rec["n_gpus"] == 2 and "one GPU" in rec["error"]


def test_two_streams_only_for_the_hero_and_the_floor():
    rc, rec = _run("--workload", "cfg1", "--streams", "2")
    assert rc != 0 and "error" in rec


def test_every_workload_kind_is_dispatched():
    src = open(BENCH).read()
    tree = ast.parse(src)
    workloads = None
    for node in ast.walk(tree):
        if isinstance(node, ast.Assign) and any(getattr(t, "id", None) == "WORKLOADS" for t in node.targets):
            workloads = ast.literal_eval(node.value)
    assert workloads and "hero" in workloads
    assert workloads["hero"] == ("gemv", 4, 14336, 4096, 1), "the BASELINE metric's shape"
    kinds = {v[0] for v in workloads.values()}
    for kind in kinds:
        assert f'"{kind}"' in src.split("def main", 1)[1] or f"'{kind}'" in src, f"kind {kind} is not dispatched"
