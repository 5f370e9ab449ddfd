"""The C ABI from plain C: include/threadcut_hip.h compiles as C99 and a C program
linked against libthreadcut_hip.so calls the host-side entry points (no GPU
needed), as a cgo / FFI binding would."""
import os
import shutil
import subprocess

import pytest

from threadcut_amd import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))

C_PROGRAM = r"""
#include <stdio.h>
#include <string.h>
#include "threadcut_hip.h"

int main(void) {
  int64_t cached[12] = {1, 2, 3, 4, 9, 9, 9, 5, 6, 7, 8, 0};
  int64_t fresh[9] = {1, 2, 3, 4, 5, 6, 7, 8, 42};
  int64_t out[3] = {-1, -1, -1};
  int64_t strides[3] = {4096, 512, 130};   /* token stride not a multiple of 8 */
  int rc;
  printf("abi %d\n", tc_abi_version());
  printf("ok '%s'\n", tc_strerror(TC_OK));
  printf("splits %d tokens %d\n", tc_decode_num_splits(1, 8, 10240, 256, 0),
         tc_decode_split_tokens(1, 8, 10240, 256, 0));
  printf("workspace %zu\n", tc_decode_workspace_bytes(1, 8, 4, 128, 40));
  rc = tc_match_split(cached, 12, fresh, 9, 2, 1, out);
  printf("split rc %d a %lld c0 %lld c %lld\n", rc, (long long)out[0], (long long)out[1], (long long)out[2]);
  rc = tc_decode_partial((void*)16, strides, (void*)32, strides, (void*)48, strides, NULL, 1000, 1, 8, 4, 128,
                         TC_DTYPE_F16, 0.088f, 256, 4, (float*)64, (float*)80, NULL);
  printf("bad strides rc %d msg %s\n", rc, strlen(tc_last_error()) ? "set" : "empty");
  return 0;
}
"""


@pytest.mark.skipif(shutil.which("gcc") is None, reason="needs gcc")
def test_c_program_uses_the_abi(tmp_path):
    _lib.load()  # the library is built
    src = tmp_path / "abi_user.c"
    src.write_text(C_PROGRAM)
    exe = tmp_path / "abi_user"
    libdir = os.path.dirname(_lib.LIB_PATH)
    subprocess.run(["gcc", "-std=c99", "-Wall", "-Werror", "-I", os.path.join(ROOT, "include"), str(src),
                    "-o", str(exe), "-L", libdir, "-lthreadcut_hip", f"-Wl,-rpath,{libdir}"],
                   check=True, capture_output=True, text=True)
    out = subprocess.run([str(exe)], check=True, capture_output=True, text=True).stdout.splitlines()
    assert out[0] == f"abi {_lib.load().tc_abi_version()}"
    assert out[1] == f"ok '{_lib.load().tc_strerror(0).decode()}'"
    assert out[2] == "splits 40 tokens 256"
    assert out[3] == f"workspace {1 * 8 * 40 * 4 * (128 + 1) * 4}"
    # cached [1 2 3 4 | 9 9 9 | 5 6 7 8 0], fresh [1 2 3 4 5 6 7 8 42]: prefix 4, suffix 5 6 7 8 at 7.
    from oracle import match as om
    r = om.split([1, 2, 3, 4, 9, 9, 9, 5, 6, 7, 8, 0], [1, 2, 3, 4, 5, 6, 7, 8, 42], min_suffix=2)
    assert tuple(r) == (4, 7, 4)
    assert out[4] == "split rc 0 a 4 c0 7 c 4"
    assert out[5] == f"bad strides rc {_lib.TC_ERR_ALIGNMENT} msg set"


def test_c_host_program_is_built():
    """tests/c_host/tc_host (built with the library) links against it and the HIP runtime and
    rejects a bad command line before any HIP call; the GPU tests run it on the device."""
    host = os.path.join(ROOT, "tests", "c_host", "tc_host")
    assert os.access(host, os.X_OK), "run python -m threadcut_amd.build"
    r = subprocess.run([host], capture_output=True, text=True, timeout=60)
    assert r.returncode == 1 and "usage" in r.stderr
    r = subprocess.run([host, "decode", "/nonexistent"], capture_output=True, text=True, timeout=60)
    assert r.returncode == 1 and "meta.txt" in r.stderr
