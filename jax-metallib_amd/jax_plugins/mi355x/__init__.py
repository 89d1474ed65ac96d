"""jax plugin registration for the MI355X PJRT plugin.

jax discovers plugins through the ``jax_plugins`` entry-point group and calls
``initialize()``; this mirrors the reference's registration
(src/jax_plugins/silicon/__init__.py:147-200): check the platform, find the
PJRT library (``GetPjrtApi``), turn off the shardy partitioner (its sdy ops
are not read by the plugin's StableHLO front end, __init__.py:170-180), and
call ``xla_bridge.register_plugin(name, priority=500, library_path=...,
options={})``.

The PJRT library is ``libmk_pjrt.so`` (built in-tree into
jax-metallib_amd/lib by the package's build): its one exported symbol is
GetPjrtApi, a PJRT API 0.114 table (include/pjrt_c_api_mi355x.h) over the
runtime C-ABI (include/mk_runtime.h).  ``libmk_kernels.so`` next to it
carries the runtime itself and is usable without jax through
``mi355x.runtime``.
"""

import os
import sys
import warnings
from pathlib import Path

PLATFORM = "mi355x"
_LIB_NAME = "libmk_pjrt.so"
_ENV = "MK_PJRT_LIBRARY_PATH"


class MI355XPluginError(RuntimeError):
    """The plugin cannot be registered."""


def _search_paths():
    pkg = Path(__file__).resolve().parent
    root = pkg.parent.parent  # jax-metallib_amd/
    return [
        (pkg / _LIB_NAME, "package directory"),
        (root / "lib" / _LIB_NAME, "jax-metallib_amd/lib (in-tree build)"),
        (Path("/usr/local/lib") / _LIB_NAME, "/usr/local/lib"),
    ]


def find_library():
    """Path of the PJRT library, or None.  The environment variable wins."""
    env = os.environ.get(_ENV)
    if env:
        if not os.path.isfile(env):
            raise MI355XPluginError(f"{_ENV}={env} does not name a file")
        return env
    for path, _ in _search_paths():
        if path.is_file():
            return str(path)
    return None


def initialize():
    """Register the plugin with jax (called by jax's plugin discovery)."""
    if not sys.platform.startswith("linux"):
        raise MI355XPluginError(f"the MI355X plugin needs Linux with ROCm, not {sys.platform}")
    library_path = find_library()
    if library_path is None:
        searched = "\n".join(f"  - {p} ({d})" for p, d in _search_paths())
        raise MI355XPluginError(
            f"Could not find {_LIB_NAME}. Searched:\n{searched}\nSet {_ENV} to its path, or build it "
            "(python jax-metallib_amd/build.py).")
    try:
        import jax

        jax.config.update("jax_use_shardy_partitioner", False)
    except Exception as e:  # jax too old to know the flag
        warnings.warn(f"could not disable the shardy partitioner: {e}", stacklevel=2)
    try:
        from jax._src import xla_bridge as xb
    except ImportError as e:
        raise MI355XPluginError(f"cannot import jax's xla_bridge: {e}") from e
    if not hasattr(xb, "register_plugin"):
        raise MI355XPluginError("this jax has no register_plugin API")
    try:
        xb.register_plugin(PLATFORM, priority=500, library_path=library_path, options={})
    except Exception as e:
        raise MI355XPluginError(f"failed to register the {PLATFORM} plugin: {e}") from e
