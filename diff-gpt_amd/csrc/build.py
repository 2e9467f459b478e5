"""Build libdgattn.so for gfx950 with hipcc (in-tree, no torch involvement).

    python diff-gpt_amd/csrc/build.py            # incremental
    python diff-gpt_amd/csrc/build.py --force    # rebuild every object
    python diff-gpt_amd/csrc/build.py --timeline # also the measurement build

Objects go to diff-gpt_amd/csrc/_build/, the library to diff-gpt_amd/lib/.
The measurement build (lib/libdgattn_timeline.so, read by timeline.py) is the
same library with the shared-prefix decode kernel compiled with DG_TIMELINE:
its waves stamp the shader clock at their phase boundaries.
"""

from __future__ import annotations

import argparse
import concurrent.futures as cf
import os
import subprocess
import sys
from pathlib import Path

HERE = Path(__file__).resolve().parent
PKG = HERE.parent
REPO = PKG.parent
BUILD = HERE / "_build"
LIB = PKG / "lib" / "libdgattn.so"
TIMELINE_LIB = PKG / "lib" / "libdgattn_timeline.so"
SOURCES = ["dg_abi.hip", "dg_rope.hip", "dg_attn_vec.hip", "dg_attn_mfma.hip", "dg_attn_mfma_f32.hip",
           "dg_attn_shared.hip", "dg_block.hip", "dg_noalloc.hip"]
HEADERS = ["dg_common.h", "dg_rope_math.h", "dg_prefill.h", str(REPO / "include" / "dgattn.h")]

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"
CFLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-fvisibility=hidden",
    "-fhip-fp32-correctly-rounded-divide-sqrt",
    # MFMA accumulators in VGPRs: the softmax reads every score with VALU ops,
    # and AGPR-resident accumulators would need a copy each way per tile
    "-mllvm", "-amdgpu-mfma-vgpr-form",
    # packed fp32 ops are kept out of every kernel of this library
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-function",
]


def _newest(paths) -> float:
    return max(Path(p).stat().st_mtime for p in paths)


def _compile(src: str, force: bool, defines: tuple[str, ...] = (), suffix: str = "") -> Path:
    s = HERE / src
    o = BUILD / (Path(src).stem + suffix + ".o")
    deps = [s] + [HERE / h if not os.path.isabs(h) else Path(h) for h in HEADERS]
    if not force and o.exists() and o.stat().st_mtime >= _newest(deps):
        return o
    cmd = [HIPCC, *CFLAGS, *(f"-D{d}" for d in defines), "-c", str(s), "-o", str(o)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        sys.stderr.write(r.stdout + r.stderr)
        raise SystemExit(f"hipcc failed on {src}")
    return o


def _link(objs: list[Path], lib: Path, force: bool) -> None:
    if force or not lib.exists() or lib.stat().st_mtime < _newest(objs):
        tmp = lib.with_suffix(".so.tmp")
        cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objs), "-o", str(tmp)]
        r = subprocess.run(cmd, capture_output=True, text=True)
        if r.returncode != 0:
            sys.stderr.write(r.stdout + r.stderr)
            raise SystemExit("link failed")
        os.replace(tmp, lib)


def build(force: bool = False, timeline: bool = False) -> Path:
    BUILD.mkdir(exist_ok=True)
    LIB.parent.mkdir(exist_ok=True)
    with cf.ThreadPoolExecutor(max_workers=min(5, len(SOURCES))) as ex:
        objs = list(ex.map(lambda s: _compile(s, force), SOURCES))
    _link(objs, LIB, force)
    if timeline:
        shared = SOURCES.index("dg_attn_shared.hip")
        tl = list(objs)
        tl[shared] = _compile("dg_attn_shared.hip", force, ("DG_TIMELINE",), "_timeline")
        _link(tl, TIMELINE_LIB, force)
    return LIB


if __name__ == "__main__":
    ap = argparse.ArgumentParser()
    ap.add_argument("--force", action="store_true")
    ap.add_argument("--timeline", action="store_true", help="also build lib/libdgattn_timeline.so")
    args = ap.parse_args()
    print(build(force=args.force, timeline=args.timeline))
