"""The static archive libxnq.a (what a build.rs `rustc-link-lib=static=xnq`
links, in the manner of xn-core's build.rs:9-19 for its CUDA kernels): a
small C program compiled against include/xnq.h links it with the HIP runtime
and calls the C ABI.  Host-only calls, so this runs without a GPU."""
import os
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
ARCHIVE = os.path.join(ROOT, "xn_amd", "libxnq.a")
ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")

PROGRAM = r"""
#include <stdio.h>
#include <string.h>
#include "xnq.h"

int main(void) {
    xnq_qtensor* qt = NULL;
    /* unknown dtype id: rejected on the host, as mod.rs:114 does */
    xnq_status st = xnq_qtensor_upload(0, 99, NULL, 1, 256, NULL, &qt);
    printf("abi=%d q4k_type_size=%zu q4k_block=%zu status=%d null=%d err=%s\n", xnq_abi_version(),
           xnq_type_size(XNQ_Q4K), xnq_block_size(XNQ_Q4K), (int)st, qt == NULL, xnq_last_error());
    return 0;
}
"""


def test_c_program_links_the_static_archive(tmp_path):
    if not os.path.exists(ARCHIVE):
        pytest.fail("libxnq.a is not built: run __graft_entry__.build()")
    cc = shutil.which("gcc")
    if cc is None:
        pytest.skip("no C compiler")
    src = tmp_path / "use_xnq.c"
    src.write_text(PROGRAM)
    obj = tmp_path / "use_xnq.o"
    exe = tmp_path / "use_xnq"
    subprocess.run([cc, "-std=c99", "-Wall", "-Werror", "-c", str(src), "-I", os.path.join(ROOT, "include"),
                    "-o", str(obj)], check=True)
    # C program + static archive; the archive's C++ host code needs the HIP
    # runtime and the C++ standard library
    subprocess.run(["g++", str(obj), ARCHIVE, "-L", os.path.join(ROCM, "lib"), f"-Wl,-rpath,{ROCM}/lib",
                    "-lamdhip64", "-o", str(exe)], check=True)
    nm = subprocess.run(["nm", str(exe)], check=True, capture_output=True, text=True).stdout
    assert " T xnq_qtensor_matmul_t" in nm  # the entry points are in the executable, not a .so
    out = subprocess.run([str(exe)], check=True, capture_output=True, text=True, timeout=120).stdout
    assert "abi=5 q4k_type_size=144 q4k_block=256 status=1 null=1" in out, out
    assert "unknown dtype" in out, out
