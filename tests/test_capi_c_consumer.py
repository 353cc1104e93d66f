"""The C ABI from a plain C caller: include/wf_api.h compiles as C99 under -Wall -Werror, a C program
links against the built library, and its calls return the documented statuses and messages (argument
errors only: no device is touched, so this runs without a GPU)."""

import os
import shutil
import subprocess

import pytest

from waveforcing_amd import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))

C_SOURCE = r"""
#include <stdio.h>
#include <string.h>
#include "wf_api.h"

static int expect(const char* what, int got, int want, const char* needle) {
  const char* msg = wf_last_error();
  if (got != want || (needle && !strstr(msg, needle))) {
    printf("FAIL %s: status %d (want %d), message '%s'\n", what, got, want, msg);
    return 1;
  }
  return 0;
}

int main(void) {
  int bad = 0;
  int v = wf_abi_version();
  if ((v >> 16) != 1) { printf("FAIL abi version 0x%x\n", v); bad = 1; }
  /* head_dim 64 is not supported by the pack */
  bad |= expect("kv_pack head_dim", wf_fp8_kv_pack((void*)16, (void*)32, 10, 2, 64, 128, (const int32_t*)48, 1, 16,
                                                   (uint8_t*)64, (uint8_t*)80, (float*)96, (float*)112, 4, NULL),
                WF_E_SHAPE, "head_dim=64");
  /* a negative element count */
  bad |= expect("encode n<0", wf_fp8_e4m3_encode_f32(NULL, NULL, -5, NULL), WF_E_INVALID, "n=-5");
  /* a misaligned activation pointer */
  bad |= expect("act quant align", wf_act_quant_i8((const void*)18, 4, 64, 64, (int8_t*)64, (float*)128, NULL),
                WF_E_ALIGN, "16-byte aligned");
  /* a LayerNorm row wider than the row kernels take */
  bad |= expect("ln dim", wf_ln_modulate_quant((const void*)16, 4, 16392, 16392, 1e-6f, NULL, NULL, NULL, NULL, 0, 1,
                                               (void*)32, 16392, NULL, NULL, NULL),
                WF_E_SHAPE, "dim=16392");
  /* empty work is a no-op success */
  bad |= expect("attn lq=0", wf_attn_paged_fp8(NULL, 0, 12, 128, 1536, NULL, NULL, NULL, NULL, 0, 1560, NULL, 0, 0,
                                               0.088f, NULL, 1536, NULL),
                WF_OK, NULL);
  if (!bad) printf("C consumer OK\n");
  return bad;
}
"""


@pytest.mark.skipif(shutil.which("gcc") is None, reason="needs gcc")
def test_c_program_links_and_gets_documented_statuses(tmp_path):
    lib = _lib.load()  # built (raises NativeLibraryMissing otherwise)
    del lib
    src = tmp_path / "consumer.c"
    src.write_text(C_SOURCE)
    exe = tmp_path / "consumer"
    lib_dir = os.path.dirname(_lib.LIB_PATH)
    cmd = ["gcc", "-std=c99", "-Wall", "-Wextra", "-Werror", "-I", os.path.join(ROOT, "include"), str(src), "-o",
           str(exe), "-L", lib_dir, "-l:" + os.path.basename(_lib.LIB_PATH), f"-Wl,-rpath,{lib_dir}"]
    build = subprocess.run(cmd, capture_output=True, text=True)
    assert build.returncode == 0, build.stderr
    run = subprocess.run([str(exe)], capture_output=True, text=True, timeout=120)
    assert run.returncode == 0, run.stdout + run.stderr
    assert "C consumer OK" in run.stdout
