"""Executable serialization on the GPU: compile -> execute -> serialize ->
destroy -> deserialize -> execute gives bit-identical outputs (the reference's
Serialize / DeserializeAndLoad contract, src/pjrt_plugin/api/
pjrt_executable.cc:169-187, :303-340), fingerprints follow the program, and a
deserialized executable compiles nothing on its first execute in a fresh
process with the disk cache off."""

import json
import struct
import os
import subprocess
import sys

import numpy as np
import pytest

from mi355x import programs as P
from mi355x import runtime as rt
from oracle import eltwise, rowops
from oracle.bf16 import bf16_bits_to_f32, f32_to_bf16_bits

from _gpu import BF16_RTOL, F32_RTOL, assert_rel_close

pytestmark = pytest.mark.gpu

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(REPO, "jax-metallib_amd")


@pytest.fixture(scope="module")
def client():
    try:
        c = rt.Client()
    except rt.PluginError as e:
        pytest.fail(f"GPU test selected but the runtime has no device: {e}")
    yield c
    c.close()


def _execute(client, exe, arrays):
    bufs = [client.buffer(*a) if isinstance(a, tuple) else client.buffer(a) for a in arrays]
    outs, done = exe.execute(bufs)
    done.wait()
    res = [o.to_numpy() for o in outs]
    for b in bufs + outs:
        b.close()
    return res


def _cases():
    rng = np.random.default_rng(7)
    x = (rng.standard_normal((256, 512)) * np.sqrt(2)).astype(np.float32)
    a = rng.standard_normal((128, 128)).astype(np.float32)
    b = rng.standard_normal((128, 128)).astype(np.float32)
    xb = (f32_to_bf16_bits(x), rt.BF16)
    return [
        ("chain6 bf16", P.chain6(256, 512, "bf16"), [xb]),
        ("softmax f32", P.softmax(256, 512, "f32"), [x]),
        ("plumbing", P.plumbing(128), [a, b]),
    ]


def _oracle_check(name, arrays, out):
    """The deserialized executable's output against the CPU oracle."""
    if name == "chain6 bf16":
        ref = eltwise.evaluate(eltwise.CHAIN6, [bf16_bits_to_f32(arrays[0][0])], "bf16")
        assert_rel_close(bf16_bits_to_f32(out), ref, BF16_RTOL, name)
    elif name == "softmax f32":
        assert_rel_close(out, rowops.softmax(arrays[0]), F32_RTOL, name)
    else:
        a, b = arrays
        ref = np.tanh(a.astype(np.float64) @ b.astype(np.float64)).sum(axis=1)
        assert_rel_close(out, ref, F32_RTOL, name, elem=False)


@pytest.mark.parametrize("name,text,arrays", _cases(), ids=[c[0] for c in _cases()])
def test_round_trip_is_bit_identical(client, name, text, arrays):
    print(f"[serialize] {name}", flush=True)
    exe = client.compile(text)
    ref = _execute(client, exe, arrays)
    fp = exe.fingerprint
    blob = exe.serialize()
    exe.close()
    exe2 = client.deserialize(blob)
    assert exe2.fingerprint == fp and len(fp) == 16
    out = _execute(client, exe2, arrays)
    for r, o in zip(ref, out):
        assert r.dtype == o.dtype and r.shape == o.shape
        assert np.array_equal(r.view(np.uint8), o.view(np.uint8)), name
    _oracle_check(name, arrays, out[0])
    # Serializing the deserialized executable gives the same bytes.
    assert exe2.serialize() == blob
    exe2.close()


def test_fingerprints_follow_the_program(client):
    e1 = client.compile(P.softmax(64, 64, "f32"))
    e2 = client.compile(P.softmax(64, 64, "f32"))
    e3 = client.compile(P.softmax(64, 128, "f32"))
    assert e1.fingerprint == e2.fingerprint != e3.fingerprint
    for e in (e1, e2, e3):
        e.close()


def test_bad_serializations(client):
    for blob in (b"", b"garbage", b"MKEX" + b"\0" * 3):
        with pytest.raises(rt.PluginError) as e:
            client.deserialize(blob)
        assert e.value.code == rt.INVALID_ARGUMENT


_CHILD = r"""
import json, sys
import numpy as np
sys.path.insert(0, {pkg!r})
from mi355x import runtime as rt
blob = open(sys.argv[1], "rb").read()
c = rt.Client()
exe = c.deserialize(blob)
x = np.load(sys.argv[2])
b = c.buffer(x, rt.BF16)
(o,), done = exe.execute([b])
done.wait()
print(json.dumps({{"stats": rt.jit_cache_stats(), "out": o.to_numpy().tobytes().hex()}}))
"""


def test_deserialized_executable_compiles_nothing(client, tmp_path):
    """A fresh process with no disk cache loads the embedded code object."""
    text = P.chain6(128, 256, "bf16")
    x = f32_to_bf16_bits(np.random.default_rng(3).standard_normal((128, 256)).astype(np.float32))
    exe = client.compile(text)
    (ref,) = _execute(client, exe, [(x, rt.BF16)])
    blob_path, x_path = tmp_path / "exe.mkex", tmp_path / "x.npy"
    blob_path.write_bytes(exe.serialize())
    exe.close()
    np.save(x_path, x)
    env = dict(os.environ, MK_DISABLE_CACHE_PERSIST="1")
    print("[serialize] fresh-process deserialize", flush=True)
    r = subprocess.run([sys.executable, "-c", _CHILD.format(pkg=PKG), str(blob_path), str(x_path)], env=env,
                       capture_output=True, text=True, timeout=240)
    assert r.returncode == 0, r.stderr
    res = json.loads(r.stdout.strip().splitlines()[-1])
    compiles, disk_hits, _ = res["stats"]
    assert compiles == 0 and disk_hits == 0, res["stats"]
    assert bytes.fromhex(res["out"]) == ref.tobytes()
    _oracle_check("chain6 bf16", [(x, rt.BF16)], ref.reshape(128, 256))


def test_code_objects_under_another_compile_tag_are_recompiled(client, tmp_path):
    """A blob written under another hiprtc version or other options (its tag
    differs) is not trusted: the fresh process compiles the program again,
    with the same result."""
    text = P.chain6(128, 256, "bf16")
    x = f32_to_bf16_bits(np.random.default_rng(4).standard_normal((128, 256)).astype(np.float32))
    exe = client.compile(text)
    (ref,) = _execute(client, exe, [(x, rt.BF16)])
    blob = bytearray(exe.serialize())
    exe.close()
    (tlen,) = struct.unpack_from("<Q", blob, 12)
    assert blob[20:27] == b"hiprtc "
    blob[20 + tlen - 1] ^= 0x01   # another tag of the same length
    blob_path, x_path = tmp_path / "exe.mkex", tmp_path / "x.npy"
    blob_path.write_bytes(bytes(blob))
    np.save(x_path, x)
    env = dict(os.environ, MK_DISABLE_CACHE_PERSIST="1")
    print("[serialize] fresh-process deserialize, foreign tag", flush=True)
    r = subprocess.run([sys.executable, "-c", _CHILD.format(pkg=PKG), str(blob_path), str(x_path)], env=env,
                       capture_output=True, text=True, timeout=240)
    assert r.returncode == 0, r.stderr
    res = json.loads(r.stdout.strip().splitlines()[-1])
    compiles, disk_hits, _ = res["stats"]
    assert compiles == 1 and disk_hits == 0, res["stats"]
    assert bytes.fromhex(res["out"]) == ref.tobytes()
