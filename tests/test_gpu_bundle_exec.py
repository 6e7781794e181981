"""g950_exec on the reference's held post-run bundles, unchanged, on the GPU:
the command-line counterpart of `operator_exec --bundle` (a100c/runtime/main.c).

Each bundle holds the inputs and the reference path's outputs; g950_exec runs
the hot-path operator on the staged storages, checks that three independent
repeats give identical bytes, and compares its outputs with the held ones under
the corpus tolerance of the case's dtype (ops/harness/opslib/case.py:153-157).
With --write the outputs land in the file, which the Python reader then
decodes and the CPU oracle checks.
"""
import json
import shutil
import subprocess

import numpy as np
import pytest

from compiler_amd import runtime as rt
from oracle import reference as ref
from tests._fixtures import GOLDEN, INDEX, dtype_of, load, values

pytestmark = pytest.mark.gpu

EXEC = rt.PKG / "lib" / "g950_exec"
OPS = {"softmax": "softmax_kernel", "matmul": "matmul_kernel", "attention": "attention_forward_kernel"}


def op_of(case):
    for prefix, op in OPS.items():
        if case.startswith(prefix):
            return op
    raise ValueError(case)


def run(*args):
    r = subprocess.run([str(EXEC), *map(str, args)], capture_output=True, text=True, timeout=120)
    line = r.stdout.strip().splitlines()[-1] if r.stdout.strip() else "{}"
    return r.returncode, json.loads(line), r.stderr


@pytest.mark.parametrize("case", sorted(INDEX))
def test_exec_held_bundle_matches_reference_outputs(case, tmp_path):
    src = GOLDEN / case
    before = (src / "bundle.bin").read_bytes()
    rtol, atol = ref.TOLERANCES[dtype_of(case)]
    rc, status, err = run("--bundle", src, "--op", op_of(case), "--repeats", 3, "--compare", rtol, atol)
    assert rc == 0, (status, err)
    assert status["status"] == "ok" and status["repeats_all_equal"] is True
    assert status["comparison"]["status"] == "PASS"
    assert status["kernel"].startswith("g950_")
    assert (src / "bundle.bin").read_bytes() == before  # private mapping: file untouched


@pytest.mark.parametrize("case", ["softmax97-bfloat16-t1", "matmul-tail-float32-t1", "attention-float16-t1"])
def test_exec_write_back_then_oracle(case, tmp_path):
    shutil.copytree(GOLDEN / case, tmp_path / case)
    work = tmp_path / case
    out_name = {"softmax_kernel": "y_ptr", "matmul_kernel": "y_ptr",
                "attention_forward_kernel": "out_ptr"}[op_of(case)]
    # clear the held outputs so only g950_exec can have written them
    b = load(case)
    img = bytearray((work / "bundle.bin").read_bytes())
    v = b.view(out_name)
    off, size = b.storages[v.storage]
    img[off:off + size] = bytes(size)
    (work / "bundle.bin").write_bytes(bytes(img))
    rc, status, err = run("--bundle", work, "--op", op_of(case), "--write")
    assert rc == 0 and status["written"] is True, (status, err)
    from compiler_amd import bundle as bmod
    got = bmod.read(work)
    dt = dtype_of(case)
    rtol, atol = ref.TOLERANCES[dt]
    if case.startswith("softmax"):
        expect = ref.softmax(values(got, "x_ptr"))
    elif case.startswith("matmul"):
        expect = ref.matmul(values(got, "a_ptr"), values(got, "b_ptr"))
    else:
        expect = ref.attention(values(got, "q_ptr"), values(got, "k_ptr"), values(got, "v_ptr"),
                               float(got.scalar("scale")), causal=False)[0]
    ok, e = ref.isclose_verdict(values(got, out_name), expect, rtol, atol)
    assert ok, e
    assert np.any(values(got, out_name) != 0)


def test_exec_contract_refusal_is_reported():
    """A softmax bundle run as a matmul: the launcher refuses (exit 2), nothing runs."""
    rc, status, _ = run("--bundle", GOLDEN / "softmax16-float32-t1", "--op", "matmul_kernel")
    assert rc == 2 and status["status"] == "refused" and "matmul" in status["reason"]
