"""The C ABI (include/amdc_q4.h) of libamdc_q4.so, without a GPU: every
declared function is exported and bound; operators called before amdc_open
fail with a message instead of crashing; amdc_open fails cleanly where there
is no device (as the reference's "GPU without a GPU" check, Makefile:153-155);
the code object holds every kernel name the host resolves."""
import os
import re
import subprocess

import pytest

import amdc

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADERS = [os.path.join(ROOT, "include", h) for h in ("amdc_q4.h", "amdc_gguf.h")]


def declared():
    src = "".join(open(h).read() for h in HEADERS)
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    return sorted(set(re.findall(r"\b(amdc_\w+)\s*\(", src)))


def test_header_functions_exported_and_bound():
    names = declared()
    assert len(names) >= 70
    lib = amdc.lib()
    for n in names:
        assert hasattr(lib, n), n
        assert n in amdc.ABI, f"{n} not bound in amdc.ABI"
    assert set(amdc.ABI) == set(names)


def test_dynamic_symbols():
    out = subprocess.run(["nm", "-D", "--defined-only", amdc.LIB_PATH], capture_output=True, text=True, check=True).stdout
    exported = set(re.findall(r" T (amdc_\w+)", out))
    assert set(declared()) <= exported


def test_kernel_names_in_code_object():
    host = open(os.path.join(ROOT, "amd.c_amd", "csrc", "amdc_host.c")).read()
    names = re.findall(r'"(amdc_(?:quant|gemv|gemm|dots|probe|q8|chain|rmsnorm|swiglu)\w*)"', host)
    assert len(names) == 80
    blob = open(amdc.HSACO_PATH, "rb").read()
    for n in names:
        assert n.encode() in blob, n


def test_ops_before_open_fail_cleanly():
    if amdc._opened:
        pytest.skip("device already open in this process")
    L = amdc.lib()
    rc = L.amdc_gemv_q4(None, None, None, 1, 1, None, None, None)
    assert rc == 4 and b"amdc_open" in L.amdc_last_error()


def test_bad_arguments_rejected_before_launch():
    L = amdc.lib()
    # kind / shape checks run on the host after the open check; without a GPU they report not-open
    rc = L.amdc_op_gemv(7, None, None, None, 1, 1, None, None, 1, 0, 0, 0, None)
    assert rc != 0
    assert L.amdc_set_tuning(3, 0, 0, 0, 0, 0) == 1 and b"power of two" in L.amdc_last_error()
    assert L.amdc_set_tuning(0, 0, 0, 9, 0, 0) == 1
    assert L.amdc_set_tuning(0, 0, 0, 0, 0, 5) == 1
    assert L.amdc_set_tuning(0, 0, 0, 0, 0, 0) == 0


def test_open_without_gpu_fails_cleanly():
    # run in a child: a process without a GPU must get an error code, not a crash
    code = ("import sys; sys.path.insert(0, %r); import amdc\n"
            "rc = amdc.lib().amdc_open(None)\n"
            "print(rc, amdc.lib().amdc_last_error().decode())\n") % os.path.join(ROOT, "amd.c_amd")
    r = subprocess.run(["python3", "-c", code], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stderr
    rc = int(r.stdout.split()[0])
    if rc == 0:
        pytest.skip("a GPU is present here")
    assert rc == 2 and ("device" in r.stdout or "runtime" in r.stdout)
