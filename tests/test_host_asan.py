"""The host staging extension (``csrc/host_stage.cpp``) under AddressSanitizer (CPU only).

The extension writes the scheduler's per-row ints and block lists straight into a caller's buffer, so an
off-by-one in its bounds would corrupt host memory silently. Here it is compiled with ``g++
-fsanitize=address`` into a small program that embeds the Python interpreter (so the sanitizer's runtime comes
first, with no preloading), and a script drives every entry point -- lists, tuples, numpy rows, empty lists,
exact-fit and too-small buffers, ids past int32, more rows than a graph holds -- while writing into buffers with
no slack, where a one-element overrun is a heap-buffer-overflow report and a non-zero exit.
"""

import shutil
import subprocess
import sys
import sysconfig
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
SOURCE = ROOT / "lean-vllm_amd" / "csrc" / "host_stage.cpp"

DRIVER = r"""
#include <Python.h>
PyMODINIT_FUNC PyInit__hoststage();
int main(int argc, char** argv) {
  if (argc != 2) return 2;
  PyImport_AppendInittab("_hoststage", PyInit__hoststage);
  Py_Initialize();
  FILE* f = fopen(argv[1], "r");
  if (!f) return 3;
  const int rc = PyRun_SimpleFileEx(f, argv[1], 1);
  if (Py_FinalizeEx() < 0) return 4;
  return rc == 0 ? 0 : 1;
}
"""

SCRIPT = r"""
import ctypes
import random

import _hoststage as hs
import numpy as np


def exact(n):
    # a heap buffer of exactly n int32 (malloc'd by ctypes: the sanitizer guards its end); the caller keeps a
    # reference for as long as the extension may write to it
    return (ctypes.c_int32 * n)()


def addr(buf):
    return ctypes.addressof(buf)


rng = random.Random(0)
for trial in range(300):
    rows = rng.randint(1, 40)
    cached = [rng.randint(0, 9000) for _ in range(rows)]
    new = [rng.randint(1, 5) for _ in range(rows)]
    lists = []
    for r in range(rows):
        ids = [rng.randint(0, 2**31 - 1) for _ in range(rng.randint(0, 6))]
        lists.append(tuple(ids) if r % 3 == 1 else np.asarray(ids, dtype=np.int64) if r % 3 == 2 else ids)
    n = hs.count_ids(lists)
    assert n == sum(len(x) for x in lists)
    cap = 3 * rows + 1 + n
    buf = exact(cap)
    got = hs.stage_rows(cached, new, lists, addr(buf), cap)
    assert got == (rows, n, max(len(x) for x in lists)), got
    flat = [int(x) for lst in lists for x in lst]
    assert list(buf[:rows]) == cached and list(buf[rows:2 * rows]) == new
    assert list(buf[3 * rows + 1:cap]) == flat
    small = exact(cap - 1)
    try:
        hs.stage_rows(cached, new, lists, addr(small), cap - 1)
        raise SystemExit("a buffer one int short was accepted")
    except ValueError:
        pass

    bs = rows + rng.randint(0, 5)
    q = rng.randint(1, 4)
    gcap = 3 * bs + 1 + n
    gbuf = exact(gcap)
    got = hs.stage_graph_rows(cached, lists, addr(gbuf), gcap, bs, q)
    assert got[0] == rows and got[1] == n, got
    gsmall = exact(gcap - 1)
    try:
        hs.stage_graph_rows(cached, lists, addr(gsmall), gcap - 1, bs, q)
        raise SystemExit("a graph buffer one int short was accepted")
    except ValueError:
        pass

keep = exact(64)  # every call below gets a live buffer
for bad in ([[2**31]], [[-2**31 - 1]]):
    try:
        hs.stage_rows([0], [1], bad, addr(keep), 8)
        raise SystemExit("an id outside int32 was accepted")
    except OverflowError:
        pass
try:
    hs.stage_graph_rows([0] * 9, [[]] * 9, addr(keep), 64, 8, 1)
    raise SystemExit("more rows than the graph holds were accepted")
except ValueError:
    pass
try:
    hs.stage_rows([0, 1], [1], [[1], [2]], addr(keep), 16)
    raise SystemExit("mismatched row counts were accepted")
except ValueError:
    pass
assert hs.count_ids([]) == 0
print("host staging clean under the sanitizer")
"""


@pytest.mark.skipif(shutil.which("g++") is None, reason="no g++")
def test_host_staging_is_clean_under_address_sanitizer(tmp_path):
    inc = sysconfig.get_paths()["include"]
    libdir = sysconfig.get_config_var("LIBDIR")
    ldver = sysconfig.get_config_var("LDVERSION")
    if not (Path(libdir) / f"libpython{ldver}.so").exists():
        pytest.skip("no shared libpython to embed")
    (tmp_path / "driver.cpp").write_text(DRIVER)
    exe = tmp_path / "stage_asan"
    build = subprocess.run(
        ["g++", "-std=c++17", "-O1", "-g", "-fno-omit-frame-pointer", "-fsanitize=address,undefined",
         f"-I{inc}", str(SOURCE), str(tmp_path / "driver.cpp"), f"-L{libdir}", f"-lpython{ldver}",
         f"-Wl,-rpath,{libdir}", "-o", str(exe)], capture_output=True, text=True)
    assert build.returncode == 0, build.stderr[-3000:]
    (tmp_path / "drive.py").write_text(SCRIPT)
    env = {"ASAN_OPTIONS": "detect_leaks=0:abort_on_error=0:halt_on_error=1",
           "UBSAN_OPTIONS": "halt_on_error=1:print_stacktrace=1", "PYTHONHOME": sys.base_prefix,
           "PATH": "/usr/bin:/bin"}
    run = subprocess.run([str(exe), str(tmp_path / "drive.py")], capture_output=True, text=True, env=env, timeout=300)
    assert run.returncode == 0, (run.stdout[-2000:], run.stderr[-4000:])
    assert "clean under the sanitizer" in run.stdout
