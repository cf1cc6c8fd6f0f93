"""The C-ABI libraries load and export exactly what include/*.h declares, and
the loader keeps the reference loader's fallback rules (no GPU needed: no
compute entry is called here)."""
import ctypes as C
import os
import re
import subprocess
import sys
import textwrap

import pytest

from sabrewing_amd import backend as B

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def header_functions(path):
    src = open(path).read()
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    return set(re.findall(r"\b((?:lag|coli|ink)_(?:hip|cuda)_\w+|sabrewing_loader_\w+)\s*\(", src))


def exported(path):
    out = subprocess.run(["nm", "-D", "--defined-only", path], stdout=subprocess.PIPE, text=True, check=True).stdout
    return {l.split()[-1] for l in out.splitlines() if " T " in l}


def test_hip_library_exports_header():
    assert os.path.exists(B.LIB_PATH), "libsabrewing_hip.so not built"
    decl = header_functions(os.path.join(ROOT, "include", "sabrewing_hip.h"))
    assert decl == set(B.EXPORTS)
    missing = decl - exported(B.LIB_PATH)
    assert not missing, missing
    lib = C.CDLL(B.LIB_PATH)                   # loads without a GPU
    for name in decl:
        assert hasattr(lib, name)


def test_coli_library_exports_header():
    """every slot of the coli table (c/backend_cuda.h:28-169) is exported and bound"""
    from sabrewing_amd.coli import COLI_EXPORTS
    decl = header_functions(os.path.join(ROOT, "include", "sabrewing_coli.h"))
    assert decl == set(COLI_EXPORTS) and len(decl) == 46
    assert not decl - exported(B.LIB_PATH)


def test_loader_exports_header():
    from sabrewing_amd.coli import COLI_EXPORTS
    decl = header_functions(os.path.join(ROOT, "include", "sabrewing_loader.h"))
    coli = {n.replace("coli_hip_", "coli_cuda_") for n in COLI_EXPORTS}
    assert decl == set(B.LOADER_EXPORTS) | coli | {"sabrewing_loader_coli_available"} | set(B.INK_EXPORTS)
    assert not decl - exported(B.LOADER_PATH)
    # the reference's own coli_cuda_* declarations (c/backend_cuda.h) are exactly these
    ref = "/root/reference/c/backend_cuda.h"
    if os.path.exists(ref):
        assert set(re.findall(r"\b(coli_cuda_\w+)\s*\(", open(ref).read())) == coli
    # and its ink_cuda_* declarations (c/backend_cuda_ink.h) these eight
    ref = "/root/reference/c/backend_cuda_ink.h"
    if os.path.exists(ref):
        assert set(re.findall(r"\b(ink_cuda_\w+)\s*\(", open(ref).read())) == set(B.INK_EXPORTS[:-1])


LOADER_PROBE = textwrap.dedent("""
    import ctypes as C, sys
    L = C.CDLL(sys.argv[1])
    L.lag_cuda_upload.restype = C.c_void_p
    L.sabrewing_loader_path.restype = C.c_char_p
    L.lag_cuda_free_bytes.restype = C.c_size_t
    L.coli_cuda_expert_group_take.restype = C.c_void_p
    L.coli_cuda_pipe_alloc.restype = C.c_void_p
    L.ink_cuda_upload.restype = C.c_void_p
    L.ink_cuda_free_bytes.restype = C.c_size_t
    print(L.sabrewing_loader_available(), L.lag_cuda_init(0), L.lag_cuda_upload(None, 16),
          L.lag_cuda_free_bytes(), L.lag_cuda_matmul_q8(None, None, None, 1, 1, 1),
          L.sabrewing_loader_path().decode(),
          L.sabrewing_loader_coli_available(), L.coli_cuda_device_count(), L.coli_cuda_device_at(0),
          L.coli_cuda_expert_group_take(0), L.coli_cuda_pipe_alloc(0, 16), L.coli_cuda_tensor_device(None),
          L.sabrewing_loader_ink_available(), L.ink_cuda_init(0), L.ink_cuda_upload(None, 16),
          L.ink_cuda_free_bytes(), L.ink_cuda_matmul_bf16(None, None, None, 1, 1, 1),
          L.ink_cuda_matmul_q8(None, None, None, None, 1, 1, 1))
""")


def run_probe(env_lib):
    env = dict(os.environ)
    env["SABREWING_HIP_LIB"] = env_lib
    r = subprocess.run([sys.executable, "-c", LOADER_PROBE, B.LOADER_PATH], env=env,
                       stdout=subprocess.PIPE, stderr=subprocess.PIPE, text=True, check=True)
    return r.stdout.split(), r.stderr


def test_loader_unavailable_sentinels(tmp_path):
    # no backend library at the configured path: every wrapper answers "not initialised"
    out, _ = run_probe(str(tmp_path / "absent.so"))
    assert out[:5] == ["0", "-1", "None", "0", "-1"]
    assert out[5] == str(tmp_path / "absent.so")
    # the coli table's sentinels (c/backend_loader.c:261-512): 0 / -1 / NULL
    assert out[6:12] == ["0", "0", "-1", "None", "None", "-1"]
    # the ink table's: -1 / NULL / 0
    assert out[12:] == ["0", "-1", "None", "0", "-1", "-1"]


def test_loader_all_or_nothing(tmp_path):
    # a library that resolves only some slots is unloaded again (c/backend_loader.c:190-250)
    src = tmp_path / "partial.c"
    src.write_text("int lag_hip_init(int d){return 0;}\n")
    so = tmp_path / "libpartial.so"
    subprocess.run(["gcc", "-shared", "-fPIC", str(src), "-o", str(so)], check=True)
    out, err = run_probe(str(so))
    assert out[:2] == ["0", "-1"] and "missing symbol" in err
    assert out[12:14] == ["0", "-1"] and "inkling backend unavailable" in err


def test_loader_relative_path_refused(tmp_path):
    # a relative SABREWING_HIP_LIB is ignored (no search of the current directory);
    # the loader falls back to the library next to itself
    out, _ = run_probe("libsabrewing_hip.so")
    assert out[5] == os.path.join(os.path.dirname(B.LOADER_PATH), "libsabrewing_hip.so")


def test_noalloc_scratch_limit():
    """lag_hip_moe_forward_scratch_bytes is host arithmetic (no device): the C2 layer's
    scratch grows with S, and the largest S that fits the allocation-free forward's
    static region is the one the header and the docs state"""
    from sabrewing_amd import configs as cf
    lib = B.load_library()
    cfg = cf.C2
    one = C.c_void_p(16)                                   # any non-null pointer: nothing is read
    w = B.LagHipMoeWeights(one, one, None, one, one, one, one, one, one, one)
    d = B.desc_of(cfg)
    need = [lib.lag_hip_moe_forward_scratch_bytes(C.byref(d), C.byref(w), s) for s in range(1, 200)]
    assert all(n > 0 for n in need) and all(a < b for a, b in zip(need, need[1:]))
    cap = 24 << 20                                         # LAG_HIP_NOALLOC_SCRATCH_BYTES
    fits = max(s for s, n in zip(range(1, 200), need) if n <= cap)
    assert fits == NOALLOC_C2_MAX_S, fits
    hdr = open(os.path.join(ROOT, "include", "sabrewing_hip.h")).read()
    assert f"fits up to S = {NOALLOC_C2_MAX_S}" in hdr
    # the IDOT contract on per-row scales carves its int8 activations and f32 h as well
    d0 = B.LagHipMoeDesc(*[getattr(d, f[0]) for f in d._fields_])
    d0.gs = 0
    assert lib.lag_hip_set_q4_mode(1) == 0
    try:
        need1 = [lib.lag_hip_moe_forward_scratch_bytes(C.byref(d0), C.byref(w), s) for s in range(1, 200)]
    finally:
        lib.lag_hip_set_q4_mode(0)
    assert max(s for s, n in zip(range(1, 200), need1) if n <= cap) == NOALLOC_C2_IDOT_MAX_S
    assert f"up to S = {NOALLOC_C2_IDOT_MAX_S} with lag_hip_set_q4_mode(1)" in hdr
    bad = B.LagHipMoeDesc(*[getattr(d, f[0]) for f in d._fields_])
    bad.hidden = 100                                       # not a multiple of 128: unsupported
    assert lib.lag_hip_moe_forward_scratch_bytes(C.byref(bad), C.byref(w), 1) == 0


# the largest C2 batch that lag_hip_moe_forward_noalloc takes (default q4 mode)
NOALLOC_C2_MAX_S = 78
NOALLOC_C2_IDOT_MAX_S = 66
