"""Model integrity on the host: the library's SHA-256 (FIPS 180-4) against
Python's hashlib on the padding boundaries, streamed files and random data,
the FIPS 180-2 appendix B examples, and the SHA256SUMS check of a model
directory as scripts/verify-models.sh:17-24 runs it (`sha256sum --check
--strict`, with the manifest rules of download-models.sh:93-97, :140-148),
including sv2_dit_load refusing a directory whose manifest does not match
before it reads any weight."""
from __future__ import annotations

import hashlib

import numpy as np
import pytest


@pytest.fixture(scope="module")
def hip():
    import sv2hip
    sv2hip.load()
    return sv2hip


def test_fips_examples(hip):
    # FIPS 180-2 appendix B.1 / B.2 and the empty message
    assert hip.sha256(b"abc").hex() == "ba7816bf8f01cfea414140de5dae2223b00361a396177a9cb410ff61f20015ad"
    assert hip.sha256(b"abcdbcdecdefdefgefghfghighijhijkijkljklmklmnlmnomnopnopq").hex() == \
        "248d6a61d20638b8e5c026930c3e6039a33ce45964ff2167f6ecedd419db06c1"
    assert hip.sha256(b"").hex() == "e3b0c44298fc1c149afbf4c8996fb92427ae41e4649b934ca495991b7852b855"


def test_lengths_across_padding_boundaries(hip):
    rng = np.random.default_rng(0)
    data = rng.integers(0, 256, 1100, dtype=np.uint8).tobytes()
    for n in list(range(0, 200)) + [255, 256, 257, 511, 512, 513, 1000, 1023, 1024, 1100]:
        assert hip.sha256(data[:n]) == hashlib.sha256(data[:n]).digest(), n


def test_large_and_file(hip, tmp_path):
    rng = np.random.default_rng(1)
    data = rng.integers(0, 256, (9 << 20) + 37, dtype=np.uint8).tobytes()  # crosses the 4 MiB read pieces
    assert hip.sha256(data) == hashlib.sha256(data).digest()
    f = tmp_path / "blob.bin"
    f.write_bytes(data)
    assert hip.sha256_file(f) == hashlib.sha256(data).digest()
    e = tmp_path / "empty.bin"
    e.write_bytes(b"")
    assert hip.sha256_file(e) == hashlib.sha256(b"").digest()
    with pytest.raises(hip.Sv2Error):
        hip.sha256_file(tmp_path / "missing.bin")


def _model_dir(tmp_path, files: dict[str, bytes]):
    for name, data in files.items():
        (tmp_path / name).write_bytes(data)
    return tmp_path


def _manifest(files: dict[str, bytes], star=False, upper=False) -> str:
    lines = []
    for name, data in files.items():
        d = hashlib.sha256(data).hexdigest()
        lines.append(f"{d.upper() if upper else d} {'*' if star else ' '}{name}")
    return "\n".join(lines) + "\n"


FILES = {f"part_{i:02d}.bin": bytes([i]) * (1000 * i + 7) for i in range(12)}


@pytest.mark.parametrize("threads", [1, 4, 0])
@pytest.mark.parametrize("form", ["text", "binary", "upper"])
def test_verify_ok(hip, tmp_path, threads, form):
    d = _model_dir(tmp_path, FILES)
    (d / "SHA256SUMS").write_text(_manifest(FILES, star=form == "binary", upper=form == "upper") + "\n")
    assert hip.verify_checksums(d, threads) == len(FILES)


def test_no_manifest_is_nothing_to_check(hip, tmp_path):
    assert hip.verify_checksums(_model_dir(tmp_path, FILES)) == 0


@pytest.mark.parametrize("case, expect", [
    ("corrupt", "corrupted"),
    ("missing", "missing"),
    ("bad_digest", "invalid SHA256"),
    ("extra_field", "invalid checksum line"),
    ("slash", "unsafe file name"),
    ("dot", "unsafe file name"),
    ("empty", "lists no files"),
])
def test_verify_rejects(hip, tmp_path, case, expect):
    files = dict(FILES)
    d = _model_dir(tmp_path, files)
    text = _manifest(files)
    if case == "corrupt":
        raw = bytearray((d / "part_05.bin").read_bytes())
        raw[100] ^= 1
        (d / "part_05.bin").write_bytes(bytes(raw))
    elif case == "missing":
        (d / "part_03.bin").unlink()
    elif case == "bad_digest":
        text = text.replace(hashlib.sha256(files["part_02.bin"]).hexdigest(), "z" * 64)
    elif case == "extra_field":
        text += hashlib.sha256(b"x").hexdigest() + "  a.bin trailing\n"
    elif case == "slash":
        text += hashlib.sha256(b"x").hexdigest() + "  sub/a.bin\n"
    elif case == "dot":
        text += hashlib.sha256(b"x").hexdigest() + "  .hidden\n"
    elif case == "empty":
        text = "\n\n"
    (d / "SHA256SUMS").write_text(text)
    with pytest.raises(hip.Sv2Error) as err:
        hip.verify_checksums(d)
    assert expect in str(err.value), str(err.value)
    if case == "corrupt":
        assert "part_05.bin" in str(err.value)


def test_dit_load_refuses_a_bad_manifest(hip, tmp_path):
    """All 34 model files present, one listed with a wrong digest: the load
    fails on the checksum before any weight is read or uploaded."""
    names = ["seedvr2_dit_input", "seedvr2_dit_output"] + [f"seedvr2_dit_block_{i:02d}" for i in range(32)]
    files = {f"{n}.ncnn{ext}": f"{n}{ext}".encode() for n in names for ext in (".param", ".bin")}
    d = _model_dir(tmp_path, files)
    text = _manifest(files)
    (d / "seedvr2_dit_block_17.ncnn.bin").write_bytes(b"tampered")
    (d / "SHA256SUMS").write_text(text)
    with pytest.raises(hip.Sv2Error) as err:
        hip.Dit.load(d, hip.F16)
    assert "seedvr2_dit_block_17.ncnn.bin is corrupted" in str(err.value), str(err.value)


_OOM_CHILD = r"""
import ctypes, resource, sys
sys.path.insert(0, sys.argv[1])
import sv2hip
lib = sv2hip.load()
digest = (ctypes.c_ubyte * 32)()
# every mapping from here on fails: the 4 MiB read buffer cannot be allocated
with open("/proc/self/statm") as f:
    pages = int(f.read().split()[0])
size = pages * resource.getpagesize()
resource.setrlimit(resource.RLIMIT_AS, (size + (1 << 20), resource.RLIM_INFINITY))
rc = lib.sv2_sha256_file(sys.argv[2].encode(), digest)
resource.setrlimit(resource.RLIMIT_AS, (resource.RLIM_INFINITY, resource.RLIM_INFINITY))
print(rc, lib.sv2_last_error().decode())
"""


def test_out_of_host_memory_is_an_error_code(hip, tmp_path):
    """No C++ exception leaves the C ABI: a host allocation that fails inside
    an entry point (here the read buffer of sv2_sha256_file, in a child
    process whose address space is capped) comes back as SV2_EDEVICE, the
    reference's allocation-failure code, with a message."""
    import os
    import subprocess
    import sys
    path = tmp_path / "data.bin"
    path.write_bytes(b"x" * 1000)
    pkg = os.path.dirname(hip.__file__)
    out = subprocess.run([sys.executable, "-c", _OOM_CHILD, pkg, str(path)], capture_output=True, text=True,
                         timeout=120)
    assert out.returncode == 0, out.stderr[-2000:]
    rc, msg = out.stdout.strip().split(" ", 1)
    assert int(rc) == hip.SV2_EDEVICE
    assert "sv2_sha256_file" in msg and "out of host memory" in msg


def test_strict_needs_a_manifest(hip, tmp_path):
    d = _model_dir(tmp_path, FILES)
    with pytest.raises(hip.Sv2Error) as err:
        hip.verify_checksums_strict(d)
    assert "SHA256SUMS is missing" in str(err.value)
    (d / "SHA256SUMS").write_text("")
    with pytest.raises(hip.Sv2Error):
        hip.verify_checksums_strict(d)  # an empty manifest counts as missing (verify-models.sh:22, [ -s ... ])
    (d / "SHA256SUMS").write_text(_manifest(FILES))
    assert hip.verify_checksums_strict(d, 3) == len(FILES)


DIT_NAMES = ["seedvr2_dit_input", "seedvr2_dit_output"] + [f"seedvr2_dit_block_{i:02d}" for i in range(32)]


def _dit_dir(d):
    files = {f"{n}.ncnn{ext}": f"{n}{ext}".encode() for n in DIT_NAMES for ext in (".param", ".bin")}
    d.mkdir(parents=True, exist_ok=True)
    _model_dir(d, files)
    return files


def test_dit_load_verify_modes(hip, tmp_path):
    """sv2_dit_load_ex: VERIFY_STRICT refuses a directory without SHA256SUMS
    and VERIFY_IF_PRESENT / VERIFY_STRICT a tampered file, all before any
    weight is read; VERIFY_NONE skips the hashing and goes on to read the
    (here not parseable) weights, failing there instead."""
    files = _dit_dir(tmp_path)
    with pytest.raises(hip.Sv2Error) as err:
        hip.Dit.load(tmp_path, hip.F16, verify=hip.VERIFY_STRICT)
    assert "SHA256SUMS is missing" in str(err.value)
    (tmp_path / "SHA256SUMS").write_text(_manifest(files))
    (tmp_path / "seedvr2_dit_block_05.ncnn.bin").write_bytes(b"tampered")
    for mode in (hip.VERIFY_IF_PRESENT, hip.VERIFY_STRICT):
        with pytest.raises(hip.Sv2Error) as err:
            hip.Dit.load(tmp_path, hip.F16, verify=mode)
        assert "seedvr2_dit_block_05.ncnn.bin is corrupted" in str(err.value)
    with pytest.raises(hip.Sv2Error) as err:
        hip.Dit.load(tmp_path, hip.F16, verify=hip.VERIFY_NONE)
    assert "corrupted" not in str(err.value) and "SHA256" not in str(err.value), str(err.value)


def test_model_set(hip, tmp_path):
    """scripts/verify-models.sh for the DiT: embeddings present and equal to
    the bundled copies, a strict dit_full_fp16 manifest, every DiT file."""
    bundled = tmp_path / "bundled"
    bundled.mkdir()
    emb = {"default_pos_emb.bin": b"P" * 64, "default_neg_emb.bin": b"N" * 80}
    _model_dir(bundled, emb)
    root = tmp_path / "models"
    files = _dit_dir(root / "dit_full_fp16")
    with pytest.raises(hip.Sv2Error) as err:
        hip.verify_model_set(root, bundled)
    assert "default_pos_emb.bin is missing" in str(err.value)
    _model_dir(root, emb)
    with pytest.raises(hip.Sv2Error) as err:
        hip.verify_model_set(root, bundled)
    assert "SHA256SUMS is missing" in str(err.value)
    (root / "dit_full_fp16" / "SHA256SUMS").write_text(_manifest(files))
    assert hip.verify_model_set(root, bundled) == len(files)
    assert hip.verify_model_set(root) == len(files)  # no bundled copies: presence only
    (root / "default_neg_emb.bin").write_bytes(b"N" * 79 + b"X")
    with pytest.raises(hip.Sv2Error) as err:
        hip.verify_model_set(root, bundled)
    assert "default_neg_emb.bin differs from the bundled embedding" in str(err.value)


_THREAD_CHILD = r"""
import ctypes, resource, sys
sys.path.insert(0, sys.argv[1])
import sv2hip
lib = sv2hip.load()
with open("/proc/self/statm") as f:
    pages = int(f.read().split()[0])
size = pages * resource.getpagesize()
# no room for a thread stack nor a 4 MiB read buffer: starting the workers
# and hashing both fail inside the call
resource.setrlimit(resource.RLIMIT_AS, (size + (2 << 20), resource.RLIM_INFINITY))
rc = lib.sv2_verify_checksums(sys.argv[2].encode(), 8)
resource.setrlimit(resource.RLIMIT_AS, (resource.RLIM_INFINITY, resource.RLIM_INFINITY))
print(rc, lib.sv2_last_error().decode())
"""


def test_checksum_workers_out_of_memory_is_an_error_code(hip, tmp_path):
    """Threads that cannot start and hashes that cannot allocate inside
    sv2_verify_checksums come back as an error code (a child process with its
    address space capped), not as a terminated process."""
    import os
    import subprocess
    import sys
    d = _model_dir(tmp_path, FILES)
    (d / "SHA256SUMS").write_text(_manifest(FILES))
    pkg = os.path.dirname(hip.__file__)
    out = subprocess.run([sys.executable, "-c", _THREAD_CHILD, pkg, str(d)], capture_output=True, text=True,
                         timeout=120)
    assert out.returncode == 0, (out.returncode, out.stderr[-2000:])
    rc, msg = out.stdout.strip().split(" ", 1)
    assert int(rc) == hip.SV2_EDEVICE, (rc, msg)
    assert "could not be hashed" in msg or "out of host memory" in msg, msg
