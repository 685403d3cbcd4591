"""$OGN_LIB: the package loads the library from that path, and the torch
extension (linked against libogn_hip.so) binds to that same copy, so every
route into the library -- ctypes and the extension -- shares one instance
(one kept-layout registry, one set of launch timings).  CPU only: it loads
the library and inspects the process's mappings, no device calls."""

import os
import shutil
import subprocess
import sys
from pathlib import Path

ROOT = Path(__file__).resolve().parent.parent
PKG = ROOT / "ops-gnn_amd"

PROBE = r"""
import sys
sys.path.insert(0, sys.argv[1])
import ops_gnn
from ops_gnn import _lib, torch_sparse_spmm  # noqa: F401  (loads the extension)
maps = [l.split()[-1] for l in open('/proc/self/maps') if l.rstrip().endswith('libogn_hip.so')]
print('\n'.join(sorted(set(maps))))
"""


def test_extension_uses_the_overridden_library(tmp_path):
    lib = PKG / "ops_gnn" / "libogn_hip.so"
    copy_dir = tmp_path / "alt"
    copy_dir.mkdir()
    shutil.copy2(lib, copy_dir / "libogn_hip.so")
    env = dict(os.environ, OGN_LIB=str(copy_dir / "libogn_hip.so"))
    res = subprocess.run([sys.executable, "-c", PROBE, str(PKG)], env=env, capture_output=True, text=True,
                         timeout=300)
    assert res.returncode == 0, res.stderr[-2000:]
    mapped = res.stdout.split()
    assert mapped == [str(copy_dir / "libogn_hip.so")], mapped
