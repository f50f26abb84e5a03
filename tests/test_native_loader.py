"""Loader failure modes, mirroring /root/reference/tests/test_native_loader.py:9-51.

The reference fakes ``tvm_ffi``; here the C-ABI library itself is faked: a
missing file, a file the dynamic loader rejects, a library that lacks an
export, and one with the wrong ABI version. Each must yield
NativeModuleUnavailable with an explanatory message.
"""

import shutil
import subprocess

import pytest

from muspace_amd.runtime import native


@pytest.fixture(autouse=True)
def _fresh_loader():
    native.load_native_module.cache_clear()
    native.native_module_proxy.cache_clear()
    yield
    native.load_native_module.cache_clear()
    native.native_module_proxy.cache_clear()


def _point_loader_at(monkeypatch, root):
    monkeypatch.setattr(native, "files", lambda package: root)


def test_missing_library_is_explained(monkeypatch, tmp_path):
    _point_loader_at(monkeypatch, tmp_path / "missing")
    assert "native library is missing" in native.native_error()
    assert not native.native_available()


def test_load_failure_is_explained(monkeypatch, tmp_path):
    library = tmp_path / native.LIBRARY_RELPATH
    library.parent.mkdir(parents=True)
    library.write_bytes(b"not an ELF file")
    _point_loader_at(monkeypatch, tmp_path)
    assert "unable to load muSPACE native library" in native.native_error()


def _build_fake_library(tmp_path, body: str):
    cc = shutil.which("gcc") or shutil.which("cc")
    if cc is None:
        pytest.skip("no C compiler to build a fake library")
    src = tmp_path / "fake.c"
    src.write_text(body)
    library = tmp_path / native.LIBRARY_RELPATH
    library.parent.mkdir(parents=True, exist_ok=True)
    subprocess.run([cc, "-shared", "-fPIC", "-o", str(library), str(src)], check=True)
    return library


def test_missing_export_is_explained(monkeypatch, tmp_path):
    _build_fake_library(tmp_path, "int muspace_abi_version(void) { return 1; }\n")
    _point_loader_at(monkeypatch, tmp_path)
    with pytest.raises(native.NativeModuleUnavailable, match="does not export 'muspace_last_error'"):
        native.native_function("ms_deform_attn_forward")


def test_abi_version_mismatch_is_explained(monkeypatch, tmp_path):
    stubs = "\n".join(
        f"int {name}(void) {{ return 0; }}"
        for name in native._EXPORTS
        if name not in ("muspace_abi_version", "muspace_last_error")
    )
    _build_fake_library(
        tmp_path,
        "int muspace_abi_version(void) { return 999; }\n"
        'const char *muspace_last_error(void) { return ""; }\n' + stubs + "\n",
    )
    _point_loader_at(monkeypatch, tmp_path)
    with pytest.raises(native.NativeModuleUnavailable, match="ABI version 999"):
        native.load_native_module()


def test_nonzero_return_code_becomes_runtime_error(monkeypatch, tmp_path):
    stubs = "\n".join(
        f"int {name}(void) {{ return 1; }}"
        for name in native._EXPORTS
        if name not in ("muspace_abi_version", "muspace_last_error")
    )
    _build_fake_library(
        tmp_path,
        f"int muspace_abi_version(void) {{ return {native.ABI_VERSION}; }}\n"
        'const char *muspace_last_error(void) { return "simulated: batch is not divisible"; }\n'
        + stubs + "\n",
    )
    _point_loader_at(monkeypatch, tmp_path)
    lib = native.load_native_module()
    with pytest.raises(RuntimeError, match="simulated: batch is not divisible"):
        lib._raise_on(lib.raw("add_one")(None, None, 4, None), "add_one")


def test_unknown_export_name_is_explained():
    lib = native.load_native_module()
    with pytest.raises(native.NativeModuleUnavailable, match="does not export 'missing_op'"):
        lib.function("missing_op")
