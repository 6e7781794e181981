"""Copy the reference's held post-run bundles for the hot-path operators into
``tests/golden/bundles/`` (run once, in the build container, where the
reference checkout exists).

The reference commits, per case, the ``a100-native-io/v1`` image after one run
of its own compiled operator (inputs + the outputs its path produced) and the
verdict of its comparator (``run.json``).  Those are data -- inputs and
expected outputs -- and are copied byte for byte; nothing of the reference's
source travels.  Source directory:
docs/compiler-agent/optimizations/k3-a100-assembly-20261111/validation/
final-metrics/candidate/<case>/pair-0/r1/{bundle/bundle.bin,bundle/bundle.json,run.json}
"""
from __future__ import annotations

import json
import shutil
import sys
from pathlib import Path

ROOT = Path("/root/reference/docs/compiler-agent/optimizations/"
            "k3-a100-assembly-20261111/validation/final-metrics/candidate")
CASES = [
    "softmax16-float32-t1", "softmax16-float16-t1", "softmax16-bfloat16-t1",
    "softmax97-float32-t1", "softmax97-float16-t1", "softmax97-bfloat16-t1",
    "matmul16-float32-t1", "matmul16-float16-t1", "matmul16-bfloat16-t1",
    "matmul128-float32-t1", "matmul128-float16-t1", "matmul128-bfloat16-t1",
    "matmul-tail-float32-t1", "matmul-tail-float16-t1", "matmul-tail-bfloat16-t1",
    "matmul256-float16-t1",
    "attention-float32-t1", "attention-float16-t1", "attention-bfloat16-t1",
]


def main(dest: Path) -> None:
    dest.mkdir(parents=True, exist_ok=True)
    index = {}
    for case in CASES:
        src = ROOT / case / "pair-0" / "r1"
        out = dest / case
        out.mkdir(exist_ok=True)
        shutil.copyfile(src / "bundle" / "bundle.bin", out / "bundle.bin")
        shutil.copyfile(src / "bundle" / "bundle.json", out / "bundle.json")
        run = json.loads((src / "run.json").read_text())
        index[case] = {"comparison": run["comparison"],
                       "runtime_status": run["runtime"]["status"],
                       "threads": run["runtime"]["threads"]}
    (dest / "index.json").write_text(json.dumps(index, indent=1, sort_keys=True) + "\n")


if __name__ == "__main__":
    main(Path(sys.argv[1]) if len(sys.argv) > 1 else Path(__file__).parent / "bundles")
