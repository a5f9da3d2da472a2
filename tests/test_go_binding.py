"""CPU checks of the Go side of the boundary (go/pkg/engine/paged_hip.go and
its no-HIP twin), the cgo binding a maintainer drops next to go-infer's
c_bridge_cgo.go.  Go is not installed here, so the checks cover what a Go
build would hand to the C compiler and the linker:

  * the cgo preamble (the comment before import "C", #cgo lines removed, as
    cgo does) compiles as C99 with -pedantic against include/goinfer_paged.h,
    and every C function the Go file calls resolves in libgoinfer_paged.so;
  * every C constant it names exists;
  * the twin (//go:build !(linux && cgo && rocm)) declares the same exported
    functions and methods with the same parameters, so builds without HIP
    keep compiling (c_bridge_nocgo.go / metal_fallback.go do the same);
  * a plain C99 program (tests/c/abi_smoke.c) links and runs the host-only
    allocator through the reference's paged_kv_test.go:7-40.
"""
import os
import re
import subprocess

import pytest

from conftest import ROOT

GO = os.path.join(ROOT, "go", "pkg", "engine")
HIP_GO = os.path.join(GO, "paged_hip.go")
NOHIP_GO = os.path.join(GO, "paged_hip_nohip.go")
INC = os.path.join(ROOT, "include")
LIBDIR = os.path.join(ROOT, "go-infer_amd")


def preamble(src):
    m = re.search(r"/\*(.*?)\*/\s*import \"C\"", src, flags=re.S)
    assert m, "no cgo preamble"
    return "\n".join(ln for ln in m.group(1).splitlines() if not ln.strip().startswith("#cgo"))


def c_names(src):
    """C identifiers the Go code uses: functions (called) and constants."""
    body = src[src.index('import "C"'):]
    funcs = sorted(set(re.findall(r"\bC\.(gi_[a-z0-9_]+)\s*\(", body)))
    consts = sorted(set(re.findall(r"\bC\.(GI_[A-Z0-9_]+)\b", body)))
    return funcs, consts


def exported_api(src):
    """Exported top-level functions and HIPPagedKV methods with their
    parameter lists (whitespace-normalised)."""
    sigs = {}
    for m in re.finditer(r"^func (\(p \*HIPPagedKV\) )?([A-Z]\w*)\((.*?)\)", src, flags=re.S | re.M):
        params = " ".join(m.group(3).split())
        sigs[("HIPPagedKV." if m.group(1) else "") + m.group(2)] = params
    return sigs


def compile_and_run(tmp_path, name, source, run=True):
    c = tmp_path / (name + ".c")
    c.write_text(source)
    exe = tmp_path / name
    cmd = ["gcc", "-std=c99", "-pedantic", "-Wall", "-Wextra", "-Werror", "-I" + INC, str(c),
           "-L" + LIBDIR, "-lgoinfer_paged", "-Wl,-rpath," + LIBDIR, "-o", str(exe)]
    r = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    assert r.returncode == 0, r.stdout
    if run:
        r = subprocess.run([str(exe)], stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True,
                           timeout=60)
        assert r.returncode == 0, r.stdout
        return r.stdout
    return ""


def test_build_tags_pair():
    hip = open(HIP_GO).read().splitlines()[0]
    nohip = open(NOHIP_GO).read().splitlines()[0]
    assert hip == "//go:build linux && cgo && rocm"
    assert nohip == "//go:build !(linux && cgo && rocm)"


def test_twin_declares_the_same_api():
    a = exported_api(open(HIP_GO).read())
    b = exported_api(open(NOHIP_GO).read())
    assert a == b
    for name in ("NewHIPPagedKV", "HIPPagedKV.Write", "HIPPagedKV.Get", "HIPPagedKV.AttentionGQA",
                 "HIPPagedKV.AttentionGQABatch", "HIPPagedKV.CopyPages", "HIPPagedKV.Close"):
        assert name in a


def test_cgo_preamble_compiles_and_links(gi, tmp_path):
    src = open(HIP_GO).read()
    pre = preamble(src)
    funcs, consts = c_names(src)
    assert "gi_paged_decode_attention" in funcs and "gi_paged_append" in funcs
    # every function cgo would reference must be one the header declares
    from test_abi import declared_functions
    assert set(funcs) <= set(declared_functions())
    prog = pre + "\n\ntypedef void (*fnp)(void);\n"
    prog += "static const fnp used[] = {\n" + ",\n".join("    (fnp)%s" % f for f in funcs) + "\n};\n"
    prog += "static const int consts[] = {" + ", ".join(consts) + "};\n"
    prog += ("int main(void)\n{\n    size_t i;\n    for (i = 0; i < sizeof used / sizeof used[0]; i++)\n"
             "        if (!used[i])\n            return 1;\n"
             "    return sizeof consts / sizeof consts[0] == %dU ? 0 : 2;\n}\n" % len(consts))
    compile_and_run(tmp_path, "cgo_preamble", prog)


def test_c99_host_runs_the_allocator(gi, tmp_path):
    out = compile_and_run(tmp_path, "abi_smoke", open(os.path.join(ROOT, "tests", "c", "abi_smoke.c")).read())
    assert "abi_smoke ok" in out
