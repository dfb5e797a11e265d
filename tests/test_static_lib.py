"""The static library (summa_amd/libsumma_amd.a, what a Rust build.rs links)
links with the plain host linker plus the HIP runtime and serves the C ABI:
a C program built against include/summa_amd.h calls host-side entry points
(no GPU needed) and gets the documented results and error messages."""
import shutil
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
ARCHIVE = ROOT / "summa_amd" / "libsumma_amd.a"

PROGRAM = r"""
#include <stdio.h>
#include "summa_amd.h"
int main(void) {
  sm_q4_gemv_job jobs[2] = {{(void*)4096, (void*)8192, (void*)16384, (void*)32768, 40, 256,
                             SM_EPI_STORE_F32, -1},
                            {(void*)4096, (void*)8192, (void*)16384, (void*)32768, 16, 128,
                             SM_EPI_STORE_F32, -1}};
  long long blocks = (long long)sm_q4_gemv_multi_plan(jobs, 2, 0);
  int st = sm_linear_cross_entropy((const float*)16, (const float*)16, 0, (const int*)16, 4, 8,
                                   16, 16, 0, 0, (float*)16, 0, (void*)(1 << 20), 1 << 20, 0);
  printf("%d %lld %d %d|%s\n", sm_version(), blocks, jobs[1].first_block, st, sm_last_error());
  return 0;
}
"""


def test_static_archive_links_with_host_linker(tmp_path):
    if not ARCHIVE.exists():
        pytest.fail("libsumma_amd.a not built (python -m summa_amd.build)")
    cc = shutil.which("gcc") or shutil.which("cc")
    src = tmp_path / "main.c"
    src.write_text(PROGRAM)
    exe = tmp_path / "main"
    subprocess.run([cc, "-I", str(ROOT / "include"), str(src), str(ARCHIVE), "-L/opt/rocm/lib",
                    "-lamdhip64", "-lstdc++", "-lm", "-Wl,-rpath,/opt/rocm/lib", "-o", str(exe)],
                   check=True, capture_output=True, text=True)
    out = subprocess.run([str(exe)], check=True, capture_output=True, text=True,
                         timeout=60).stdout.strip()
    head, msg = out.split("|", 1)
    version, blocks, first, st = map(int, head.split())
    assert version >= 1 and blocks == 3 + 1 and first == 3 and st == -1
    assert msg == "linear cross-entropy chunk size must be positive"
