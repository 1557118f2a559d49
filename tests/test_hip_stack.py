"""CPU tests of which HIP runtime and which hipBLASLt the libraries bind to in one process.

PyTorch's ROCm wheel bundles a HIP runtime (ROCm 7.0) and an older hipBLASLt and rocRoller
under the same sonames as the ROCm installation's (7.2), whose headers libdadgpt_gen was
compiled against. Importing dadgpt_amd before torch must leave one HIP runtime (PyTorch's) and
two hipBLASLt stacks side by side: the ROCm one for these libraries, PyTorch's for PyTorch.
Each check runs in a fresh interpreter (import order matters); none touches a GPU.
"""
import os
import re
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIBS = [os.path.join(ROOT, "dadgpt_amd", "lib", n) for n in ("libdadgpt_attn.so",
                                                           "libdadgpt_gen.so")]

PROBE = r"""
import re, sys
sys.path.insert(0, {root!r})
{first}
{second}
import dadgpt_amd
maps = open("/proc/self/maps").read()
names = sorted(set(re.findall(r"(\S*/lib(?:hipblaslt|rocroller|amdhip64)\S*)", maps)))
print("LOAD_ERROR", repr(dadgpt_amd.load_error))
for n in names:
    print("MAPPED", n)
"""


def _run(first, second):
    code = PROBE.format(root=ROOT, first=first, second=second)
    r = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, r.stderr[-2000:]
    err = re.search(r"LOAD_ERROR (.*)", r.stdout).group(1)
    mapped = re.findall(r"MAPPED (\S+)", r.stdout)
    return err, mapped


def _torch_lib():
    import importlib.util
    spec = importlib.util.find_spec("torch")
    return os.path.join(list(spec.submodule_search_locations)[0], "lib")


def test_package_first_binds_both_stacks():
    err, mapped = _run("import dadgpt_amd", "import torch")
    assert err == "''", err
    tl = _torch_lib()
    runtimes = [m for m in mapped if "libamdhip64" in m]
    assert runtimes == [os.path.join(tl, "libamdhip64.so")], runtimes  # one HIP runtime
    blaslt = [m for m in mapped if "libhipblaslt" in m]
    assert any(m.startswith("/opt/rocm") for m in blaslt), blaslt   # ours
    assert os.path.join(tl, "libhipblaslt.so") in blaslt, blaslt     # PyTorch's
    roller = [m for m in mapped if "librocroller" in m]
    assert any(m.startswith("/opt/rocm") for m in roller) and len(roller) == 2, roller


def test_torch_first_is_refused_with_the_reason():
    err, _ = _run("import torch", "")
    assert "import dadgpt_amd before torch" in err, err


def _undefined_hip(path):
    out = subprocess.run(["nm", "-D", "--undefined-only", path], check=True,
                         capture_output=True, text=True).stdout
    return {re.sub(r"@.*", "", line.split()[-1]) for line in out.splitlines()
            if re.search(r"\bU hip", line)}


def test_every_hip_symbol_needed_is_in_pytorchs_runtime():
    """The process's HIP runtime is PyTorch's (7.0): every HIP entry point that these
    libraries, and the ROCm 7.2 hipBLASLt and rocRoller they open, import must exist there."""
    out = subprocess.run(["nm", "-D", "--defined-only", os.path.join(_torch_lib(),
                                                                     "libamdhip64.so")],
                         check=True, capture_output=True, text=True).stdout
    have = {re.sub(r"@.*", "", line.split()[-1]) for line in out.splitlines()}
    for path in LIBS + ["/opt/rocm/lib/libhipblaslt.so.1", "/opt/rocm/lib/librocroller.so.1"]:
        if not os.path.exists(path):
            pytest.skip(f"{path} missing")
        missing = sorted(_undefined_hip(path) - have)
        assert not missing, (path, missing)


def test_gen_library_does_not_link_hipblaslt():
    """libhipblaslt is opened by path at run time, never resolved by soname at load time."""
    out = subprocess.run(["readelf", "-d", LIBS[1]], check=True, capture_output=True,
                         text=True).stdout
    assert "hipblaslt" not in out


def _compiled_hipblaslt():
    """The hipBLASLt version the headers declare (major*100000 + minor*100 + patch)."""
    text = open("/opt/rocm/include/hipblaslt/hipblaslt-version.h").read()
    v = {k: int(re.search(rf"HIPBLASLT_VERSION_{k}\s+(\d+)", text).group(1))
         for k in ("MAJOR", "MINOR", "PATCH")}
    return v["MAJOR"] * 100000 + v["MINOR"] * 100 + v["PATCH"]


def test_stack_pairs_accepted_and_refused():
    """dadgpt_blas_create accepts only (HIP runtime, hipBLASLt) pairs the GPU tests run on:
    HIP 7.0 (PyTorch's) or 7.2 (the ROCm installation's) with the compiled hipBLASLt."""
    from dadgpt_amd import gpt2

    lt = _compiled_hipblaslt()
    assert gpt2.blas_stack_supported(70051831, lt)
    assert gpt2.blas_stack_supported(70226015, lt)
    assert not gpt2.blas_stack_supported(70226015, lt + 1)
    assert not gpt2.blas_stack_supported(70051831, lt - 100)
    for rt in (60400000, 70100000, 70300000, 80000000, -1):
        assert not gpt2.blas_stack_supported(rt, lt), rt


CREATE_PROBE = r"""
import ctypes, sys
sys.path.insert(0, {root!r})
import dadgpt_amd
from dadgpt_amd import gpt2
import torch
v = gpt2.blas_stack_versions()
print("RUNTIME", v["hip_runtime"], v["hip_runtime_str"])
if torch.cuda.device_count() == 0:
    h = ctypes.c_void_p()
    st = gpt2.gen_lib().dadgpt_blas_create(ctypes.byref(h))
    print("CREATE", st, gpt2.last_error())
"""


def test_process_runtime_is_pytorchs_and_no_device_is_an_error():
    """With the package imported before torch, the process's HIP runtime (the one the version
    check sees) is PyTorch's 7.0; with no device, handle creation returns an error instead of
    letting hipBLASLt end the process."""
    r = subprocess.run([sys.executable, "-c", CREATE_PROBE.format(root=ROOT)],
                       capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, r.stdout + r.stderr[-2000:]
    rt = int(re.search(r"RUNTIME (-?\d+)", r.stdout).group(1))
    assert rt // 100000 == 700, rt
    m = re.search(r"CREATE (\d+) (.*)", r.stdout)
    if m:
        assert m.group(1) == "3" and "no HIP device" in m.group(2), r.stdout
