"""The C ABI from C: tests/c/abi_check.c (include/sas.h, linked to
libsas.so, no Python in between) runs the bit-exact scheduler on every
reference fixture (written by importing the reference metadata.py, see
tests/golden/make_metadata_fixtures.py) and the host-side argument errors of
every entry point. CPU only: no device memory is touched."""

from __future__ import annotations

import json
import os
import shutil
import subprocess

import pytest

from dsv4_amd import _lib

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)

# defaults of sparse_attn_sharedkv_metadata (metadata.py:1018-1045)
DEFAULTS = dict(num_heads_kv=1, batch_size=0, max_seqlen_q=0, max_seqlen_kv=0, ori_topk=0, cmp_topk=0,
                cmp_ratio=-1, ori_mask_mode=4, cmp_mask_mode=3, ori_win_left=127, ori_win_right=0,
                layout_q="BSND", layout_kv="PA_ND", has_ori_kv=True, has_cmp_kv=True,
                aic_core_num=24, aiv_core_num=48)


def _line(name, kw):
    k = dict(DEFAULTS, **kw)
    arr = lambda a: f"{len(a or [])} " + " ".join(str(int(x)) for x in (a or []))  # noqa: E731
    head = [k["num_heads_q"], k["num_heads_kv"], k["head_dim"], k["batch_size"], k["max_seqlen_q"],
            k["max_seqlen_kv"], k["ori_topk"], k["cmp_topk"], k["cmp_ratio"], k["ori_mask_mode"],
            k["cmp_mask_mode"], k["ori_win_left"], k["ori_win_right"]]
    tail = [int(bool(k["has_ori_kv"])), int(bool(k["has_cmp_kv"])), k["aic_core_num"], k["aiv_core_num"]]
    return " ".join([name] + [str(int(x)) for x in head] + [k["layout_q"], k["layout_kv"]] +
                    [str(x) for x in tail] + [arr(k.get("cu_seqlens_q")), arr(k.get("seqused_kv")),
                                              arr(k.get("seqused_q"))])


@pytest.fixture(scope="module")
def abi_check(tmp_path_factory):
    gcc = shutil.which("gcc")
    if gcc is None or not os.path.exists(_lib.LIB_PATH):
        pytest.skip("gcc or libsas.so missing")
    exe = str(tmp_path_factory.mktemp("cabi") / "abi_check")
    lib_dir = os.path.dirname(_lib.LIB_PATH)
    subprocess.run([gcc, "-std=c99", "-O1", "-Wall", "-Werror", "-I", os.path.join(ROOT, "include"),
                    os.path.join(HERE, "c", "abi_check.c"), "-o", exe, "-L", lib_dir, "-lsas",
                    f"-Wl,-rpath,{lib_dir}"], check=True)
    return exe


def test_c_caller_matches_fixtures_and_errors(abi_check):
    with open(os.path.join(HERE, "golden", "metadata_fixtures.json")) as f:
        cases = json.load(f)["cases"]
    text = "\n".join(_line(c["name"], c["kwargs"]) for c in cases) + "\nEND\n"
    res = subprocess.run([abi_check], input=text, capture_output=True, text=True, timeout=120)
    lines = res.stdout.strip().splitlines()
    assert res.returncode == 0 and lines[-1] == "ABI ok", res.stdout[-500:] + res.stderr[-500:]
    got = {ln.split()[0]: [int(x) for x in ln.split()[1:]] for ln in lines[:-1]}
    assert len(got) == len(cases)
    for c in cases:
        rc, vals = got[c["name"]][0], got[c["name"]][1:]
        assert rc == 0, c["name"]
        expected = [0] * 1024
        for i, v in c["nonzero"]:
            expected[i] = v
        assert vals == expected, c["name"]
