"""Runs the Node-side suites (tests/node/*.test.mjs) through tests/node/run.mjs:
the package's TypeScript op API over the Node-API addon, checked against the
ECMAScript oracle on the reference's own test inputs."""
import os
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
NODE = shutil.which("node")
ADDON = os.path.join(ROOT, "web-xpu-ops_amd", "lib", "wxo_q8.node")


def run(mode):
    proc = subprocess.run([NODE, os.path.join(ROOT, "tests", "node", "run.mjs"), mode],
                          capture_output=True, text=True, timeout=300)
    print(proc.stdout[-6000:], proc.stderr[-2000:])
    return proc


@pytest.mark.skipif(NODE is None, reason="node not on PATH")
def test_node_suite_cpu():
    assert os.path.exists(ADDON), "run __graft_entry__.build() first"
    proc = run("cpu")
    assert proc.returncode == 0, proc.stdout[-3000:]
    assert " 0 failed" in proc.stdout


@pytest.mark.gpu
@pytest.mark.timeout(400)
@pytest.mark.skipif(NODE is None, reason="node not on PATH")
def test_node_suite_gpu():
    proc = run("gpu")
    assert proc.returncode == 0, proc.stdout[-3000:]
    assert " 0 failed" in proc.stdout and " 0 passed" not in proc.stdout
