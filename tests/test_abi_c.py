"""A C program compiled against include/czip_hip.h (tests/abi/abi_check.c)
pins the boundary's struct layouts against the ctypes mirror the Python
package uses, and calls the host-only entry points of libczip_hip.so from C.
CPU only (no compute call)."""
import ctypes as C
import os
import subprocess

import pytest

from conftest import MODEL_PATH, ROOT


@pytest.fixture(scope="module")
def abi_bin(tmp_path_factory):
    import czip_amd
    czip_amd.lib()  # built
    out = str(tmp_path_factory.mktemp("abi") / "abi_check")
    libdir = os.path.dirname(czip_amd.LIB_PATH)
    subprocess.check_call(["gcc", "-std=c99", "-Wall", "-Werror", "-I", os.path.join(ROOT, "include"),
                           os.path.join(ROOT, "tests", "abi", "abi_check.c"), "-o", out, "-L", libdir, "-lczip_hip",
                           f"-Wl,-rpath,{libdir}"])
    return out


def test_struct_layouts_match_the_ctypes_mirror(abi_bin):
    import czip_amd
    lines = subprocess.check_output([abi_bin, "layout"], text=True).splitlines()
    sizes = {l.split()[1]: int(l.split()[2]) for l in lines if l.startswith("sizeof")}
    mirror = {"czip_layer_desc": czip_amd.LayerDesc, "czip_model_desc": czip_amd.ModelDesc,
              "czip_container": czip_amd.ContainerInfo}
    for name, cls in mirror.items():
        assert sizes[name] == C.sizeof(cls), name
    fields = [l.split() for l in lines if not l.startswith("sizeof")]
    assert len(fields) == sum(len(c._fields_) for c in mirror.values())
    for qual, off, size in fields:
        sname, fname = qual.split(".")
        f = getattr(mirror[sname], fname)
        assert (f.offset, f.size) == (int(off), int(size)), qual


def test_host_entry_points_from_c(abi_bin, orc):
    import container as OC
    r = subprocess.run([abi_bin, "host", MODEL_PATH], capture_output=True, text=True, cwd=ROOT)
    assert r.returncode == 0, r.stdout + r.stderr
    out = dict(l.split(" ", 1) for l in r.stdout.splitlines())
    assert out["model"] == ("vocab 1024 layers 1 heads 6 kv 1 d 384 ff 1024 ctx 1024 max_seq 8192 "
                            "coef 37819 total 1073739776")
    t, _ = orc.read_czm(MODEL_PATH)
    L = f"qkv 819/20 out 819/20 score_mult0 {int(t['layers.0.attn.score_mult'][0])} " \
        f"embed00 {int(t['embed.weight'][0, 0])} lut0 {int(t['lut.exp2'][0])}"
    assert out["layer0"] == L
    assert int(out["hash"], 16) == OC.model_id_hash("models/v001_eng.czm")
    assert out["container"].startswith("ok ")
