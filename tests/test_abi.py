"""The C-ABI library: builds, loads without a GPU, exports every function that include/snl.h
declares, and does not link the oracle."""
import ctypes
import os
import re
import subprocess
import sys

import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB = os.path.join(REPO, "sense-nova-server_amd", "libsnl.so")
HEADER = os.path.join(REPO, "include", "snl.h")


@pytest.fixture(scope="module")
def libsnl():
    if not os.path.exists(LIB):
        subprocess.run([sys.executable, os.path.join(REPO, "sense-nova-server_amd", "build.py")], check=True)
    return ctypes.CDLL(LIB)


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(snl_\w+)\s*\(", text)))


def test_header_declares_the_engine_api():
    names = declared_functions()
    for f in ("snl_engine_create", "snl_forward", "snl_mtp", "snl_rollback", "snl_snapshot", "snl_restore",
              "snl_reset", "snl_gemv", "snl_deltanet", "snl_attention"):
        assert f in names


def test_every_declared_function_is_exported(libsnl):
    missing = [f for f in declared_functions() if not hasattr(libsnl, f)]
    assert not missing, missing


def test_library_does_not_link_the_oracle():
    out = subprocess.run(["readelf", "-d", LIB], capture_output=True, text=True, check=True).stdout
    needed = re.findall(r"\(NEEDED\).*\[(.*)\]", out)
    assert needed and not any("oracle" in n for n in needed), needed


def test_product_package_does_not_import_the_oracle():
    pkg = os.path.join(REPO, "sense-nova-server_amd")
    for root, _, files in os.walk(pkg):
        for f in files:
            if f.endswith((".py", ".cpp", ".hip", ".h")):
                src = open(os.path.join(root, f)).read()
                assert "import oracle" not in src and "liboracle" not in src and "snl_oracle" not in src, f
