"""Host-only checks of executable serialization and the compile cache (no GPU
needed: hiprtc compiles gfx950 code objects on the CPU).

The reference serializes an executable as its program and recompiles it on
load (src/pjrt_plugin/api/pjrt_executable.cc:169-187, :303-340); its tests
only round-trip through jax.  Here the layout written in include/mk_runtime.h
is parsed independently below, every malformed variant must fail with
INVALID_ARGUMENT (the reference's code for empty data, :304-306), and the
disk cache is exercised in fresh processes so the in-memory cache cannot
answer for it."""

import json
import os
import struct
import subprocess
import sys

import pytest

from mi355x import programs as pg
from mi355x import runtime as rt

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(REPO, "jax-metallib_amd")


def _parse(blob):
    """The documented layout, read independently of the library."""
    assert blob[:4] == b"MKEX"
    ver, flags, tlen = struct.unpack_from("<IIQ", blob, 4)
    off = 20
    tag = blob[off:off + tlen]
    off += tlen
    (plen,) = struct.unpack_from("<Q", blob, off)
    off += 8
    program = blob[off:off + plen]
    off += plen
    (n,) = struct.unpack_from("<I", blob, off)
    off += 4
    objs = []
    for _ in range(n):
        (sl,) = struct.unpack_from("<Q", blob, off)
        src = blob[off + 8:off + 8 + sl]
        off += 8 + sl
        (cl,) = struct.unpack_from("<Q", blob, off)
        code = blob[off + 8:off + 8 + cl]
        off += 8 + cl
        objs.append((src, code))
    assert off == len(blob)
    return ver, flags, tag, program, objs


def test_serialized_layout_and_code_objects(tmp_path, monkeypatch):
    monkeypatch.setenv("MK_CACHE_DIR", str(tmp_path))
    text = pg.chain6(256, 256, "bf16")
    blob = rt.serialize_program(text)
    ver, flags, tag, program, objs = _parse(blob)
    assert (ver, flags) == (2, 0)
    # The compile tag names the hiprtc version and the options.
    assert tag.startswith(b"hiprtc ") and b"--offload-arch=gfx950" in tag and b"-ffp-contract=off" in tag
    assert program == text.encode()
    assert len(objs) == 1
    src, code = objs[0]
    assert b"mk_ew_jit" in src and code[:4] == b"\x7fELF"
    assert rt.inspect_serialized(blob) == (len(text.encode()), 1)
    # A program with no elementwise step carries no code object.
    blob2 = rt.serialize_program(pg.matmul(64, 64, 64))
    assert rt.inspect_serialized(blob2)[1] == 0


def _expect_invalid(blob):
    with pytest.raises(rt.PluginError) as e:
        rt.inspect_serialized(blob)
    assert e.value.code == rt.INVALID_ARGUMENT, e.value


def test_malformed_serializations_are_invalid_argument(tmp_path, monkeypatch):
    monkeypatch.setenv("MK_CACHE_DIR", str(tmp_path))
    blob = rt.serialize_program(pg.chain6(64, 64, "f32"))
    _expect_invalid(b"")
    _expect_invalid(b"MKEY" + blob[4:])
    _expect_invalid(blob[:4] + struct.pack("<I", 1) + blob[8:])   # the format before the tag
    _expect_invalid(blob[:4] + struct.pack("<I", 3) + blob[8:])
    _expect_invalid(blob + b"\0")
    (tlen,) = struct.unpack_from("<Q", blob, 12)
    poff = 20 + tlen
    # Every truncation point, header through the last code byte.
    for cut in sorted({1, 4, 8, 12, 19, 20, 21, poff - 1, poff, poff + 7, poff + 8, len(blob) // 2,
                       len(blob) - 1}):
        _expect_invalid(blob[:cut])
    # A tag or program length that runs past the end.
    _expect_invalid(blob[:12] + struct.pack("<Q", len(blob)) + blob[20:])
    _expect_invalid(blob[:poff] + struct.pack("<Q", len(blob)) + blob[poff + 8:])


def test_serialize_rejects_unsupported_programs():
    with pytest.raises(rt.PluginError) as e:
        rt.serialize_program("module { func.func @main() { stablehlo.frobnicate } }")
    assert e.value.code in (rt.UNIMPLEMENTED, rt.INVALID_ARGUMENT)


_CHILD = r"""
import json, sys
sys.path.insert(0, {pkg!r})
from mi355x import programs as pg, runtime as rt
blob = rt.serialize_program(pg.chain6(128, 128, "bf16"))
print(json.dumps({{"stats": rt.jit_cache_stats(), "blob": blob.hex()}}))
"""


def _child(env_extra):
    env = dict(os.environ)
    env.update(env_extra)
    out = subprocess.run([sys.executable, "-c", _CHILD.format(pkg=PKG)], env=env, capture_output=True,
                         text=True, timeout=300)
    assert out.returncode == 0, out.stderr
    r = json.loads(out.stdout.strip().splitlines()[-1])
    return tuple(r["stats"]), bytes.fromhex(r["blob"])


def test_disk_cache_across_processes(tmp_path):
    d = str(tmp_path / "cache")
    env = {"MK_CACHE_DIR": d, "MK_DISABLE_CACHE_PERSIST": "0"}
    (c1, h1, _), blob1 = _child(env)
    assert (c1, h1) == (1, 0)
    files = [f for f in os.listdir(d) if f.startswith("ew-") and f.endswith(".hsaco")]
    assert len(files) == 1 and not [f for f in os.listdir(d) if ".tmp." in f]
    (c2, h2, _), blob2 = _child(env)
    assert (c2, h2) == (0, 1), "second process must load the code object from disk"
    assert blob1 == blob2
    # A damaged cache file is ignored: compiled again and rewritten.
    path = os.path.join(d, files[0])
    with open(path, "r+b") as f:
        f.truncate(os.path.getsize(path) // 2)
    (c3, h3, _), blob3 = _child(env)
    assert (c3, h3) == (1, 0) and blob3 == blob1
    (c4, h4, _), _ = _child(env)
    assert (c4, h4) == (0, 1)


def test_disk_cache_can_be_disabled(tmp_path):
    d = str(tmp_path / "off")
    (c, h, _), _ = _child({"MK_CACHE_DIR": d, "MK_DISABLE_CACHE_PERSIST": "1"})
    assert (c, h) == (1, 0)
    assert not os.path.exists(d) or not os.listdir(d)
