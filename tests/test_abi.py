"""The C ABI library loads and exports every entry point include/wavo_hip.h declares; error paths that
need no GPU (no device, bad arguments) report through wh_last_error.  No compute without a GPU."""

import ctypes
import os
import re

import pytest

import wavo_amd as wa

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared():
    text = open(os.path.join(ROOT, "include", "wavo_hip.h")).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(wh_[a-z0-9_]+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    lib = ctypes.CDLL(wa.LIB_PATH)
    names = declared()
    assert len(names) >= 30
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, missing
    # The binding's signature table covers exactly the header.
    assert sorted(wa.SIGNATURES) == names


def test_binding_loads():
    assert wa.lib() is not None


def test_open_without_gpu_or_bad_index_is_a_gpu_error():
    # Here (no GPU) any index fails; on a GPU box an index past the devices fails the same way
    # (the reference's index_past_the_gpus, src/gpu/mod.rs:1712-1715).
    with pytest.raises(wa.WavoError) as e:
        wa.Gpu(1 << 20)
    assert e.value.fatal
    assert "GPU" in str(e.value) or "gfx950" in str(e.value)


def test_null_context_arguments_are_rejected():
    L = wa.lib()
    assert L.wh_sync(None) == wa.EARG
    assert L.wh_gemm(None, None, None, None, 1, 0, 0.0) == wa.EARG
    assert L.wh_linear_width(None) == 0
    assert L.wh_attend_len(4100, 2, 40) == 17 * 2 * 42


def test_static_library_links_a_c_program(tmp_path):
    # libwavo_hip.a, the library a host program links (the Rust shim's build script does): a C program
    # that includes the header and calls the ABI links against it with the HIP runtime alone and runs
    # (without a GPU, wh_open reports the error; on a GPU box it opens device 0).
    lib_a = os.path.join(ROOT, "wavo_amd", "libwavo_hip.a")
    assert os.path.exists(lib_a), "build the library first (__graft_entry__.build)"
    src = tmp_path / "main.c"
    src.write_text(r'''
#include <stdio.h>
#include "wavo_hip.h"
int main(void) {
  wh_ctx *ctx = NULL;
  int rc = wh_open(-1, &ctx);
  printf("limit %zu open %d %s\n", wh_gemm_noalloc_limit(), rc, rc ? wh_last_error(NULL) : "ok");
  if (!rc) wh_close(ctx);
  return 0;
}
''')
    exe = tmp_path / "main"
    import subprocess
    subprocess.run(["/opt/rocm/bin/hipcc", "--offload-arch=gfx950", "-x", "c++", str(src), "-x", "none", lib_a,
                    "-I", os.path.join(ROOT, "include"), "-o", str(exe)], check=True, capture_output=True, timeout=300)
    out = subprocess.run([str(exe)], capture_output=True, text=True, timeout=120)
    assert out.returncode == 0, out.stderr
    assert out.stdout.startswith(f"limit {32 << 20} open "), out.stdout
