"""The jax plugin entry point (jax_plugins/mi355x) fails with a clear error
when its PJRT library or jax is missing, and honours the library-path
environment variable, as the reference's initialize() does
(src/jax_plugins/silicon/__init__.py:147-200)."""

import importlib
import os
import sys

import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, os.path.join(REPO, "jax-metallib_amd"))

plugin = importlib.import_module("jax_plugins.mi355x")


def test_missing_library_is_a_clear_error(monkeypatch, tmp_path):
    monkeypatch.delenv("MK_PJRT_LIBRARY_PATH", raising=False)
    monkeypatch.setattr(plugin, "_search_paths", lambda: [(tmp_path / "libmk_pjrt.so", "tmp")])
    with pytest.raises(plugin.MI355XPluginError) as ei:
        plugin.initialize()
    assert "libmk_pjrt.so" in str(ei.value) and "MK_PJRT_LIBRARY_PATH" in str(ei.value)


def test_env_path_must_exist(monkeypatch, tmp_path):
    monkeypatch.setenv("MK_PJRT_LIBRARY_PATH", str(tmp_path / "nope.so"))
    with pytest.raises(plugin.MI355XPluginError):
        plugin.find_library()
    f = tmp_path / "libmk_pjrt.so"
    f.write_bytes(b"")
    monkeypatch.setenv("MK_PJRT_LIBRARY_PATH", str(f))
    assert plugin.find_library() == str(f)


def test_without_jax_registration_fails_loudly(monkeypatch, tmp_path):
    f = tmp_path / "libmk_pjrt.so"
    f.write_bytes(b"")
    monkeypatch.setenv("MK_PJRT_LIBRARY_PATH", str(f))
    try:
        import jax  # noqa: F401
        pytest.skip("jax is installed")
    except ImportError:
        pass
    with pytest.warns(UserWarning):
        with pytest.raises(plugin.MI355XPluginError) as ei:
            plugin.initialize()
    assert "xla_bridge" in str(ei.value)


def test_in_tree_library_is_found_and_exports_the_table(monkeypatch):
    """The in-tree build is found without the environment variable, and it is
    a loadable PJRT plugin: GetPjrtApi returns a table of API 0.114."""
    import ctypes
    monkeypatch.delenv("MK_PJRT_LIBRARY_PATH", raising=False)
    path = plugin.find_library()
    assert path and path.endswith("libmk_pjrt.so") and os.path.isfile(path)
    lib = ctypes.CDLL(path)
    lib.GetPjrtApi.restype = ctypes.POINTER(ctypes.c_size_t * 5)
    head = lib.GetPjrtApi().contents
    # struct_size, extension_start, then PJRT_Api_Version {struct_size,
    # extension_start, int major, int minor}: major/minor share one word.
    assert head[0] == 1088
    assert head[4] == (114 << 32)
