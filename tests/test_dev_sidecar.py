"""The FIDESlib .dev sidecar (cryptocontext.bin.dev) and the rotation-key loader it drives, on the CPU.

The reference client writes the sidecar next to cryptocontext.bin (writeDevSidecar,
hpc_gpu_port/mac_fhe_client.cpp:178-194): "1 { 0 }", the auto-load flags, "RotationIndexes: { ... }" (rotation
AMOUNTS: FIDESlib's LoadContext uploads GetRotationKeySwitchKey(pk, step) for each), "KeyDist: 1" and
"BootstrapSlots: { ... }".  Golden: the reference's verification kit records the SHA-256 of the sidecar its client
wrote for the r17 session (results/dense-demo-s31/sessions/demo_20260918T074952Z/verification/
MAC_KEYS_MANIFEST.sha256:4) beside the rotation contract of that session (tests/golden/contract_r17.json, 73 rotation
amounts, 65536 slots); the engine's writer must reproduce that file byte for byte.  The loader's choice of keys is
checked against part files written from the part format's specification (tests/keypart_util.py).
"""
import hashlib
import json
import os

import numpy as np
import pytest

from conftest import GOLDEN
from engine_loader import load_ckks
from keypart_util import part_bytes

# sha256 of cryptocontext.bin.dev in the r17 session's key manifest (MAC_KEYS_MANIFEST.sha256:4)
R17_DEV_SHA256 = "adf730e09fb5227508e6160fa000cea1fdc7b1f90a4d08ad35e8d3afda3c9f89"
R17_DEV_BYTES = 361  # its size in the session's key listing (pod_pull/sovereignty_r17.log:11)


@pytest.fixture(scope="module")
def ckks():
    return load_ckks()


def contract():
    with open(os.path.join(GOLDEN, "contract_r17.json")) as f:
        return json.load(f)


def test_writer_reproduces_the_reference_sidecar(ckks, tmp_path):
    c = contract()
    rots = sorted(set(c["rotationAmounts"]))   # the client sorts and dedups them (mac_fhe_client.cpp:442-443)
    path = str(tmp_path / "cryptocontext.bin.dev")
    ckks.dev_sidecar_write(path, rots, [c["slots"]])
    data = open(path, "rb").read()
    assert len(data) == R17_DEV_BYTES
    assert hashlib.sha256(data).hexdigest() == R17_DEV_SHA256
    got = ckks.dev_sidecar_read(path)
    assert got == {"devices": [0], "AutoLoadCiphertexts": 1, "AutoLoadPlaintexts": 0, "KeyDist": 1,
                   "RotationIndexes": rots, "BootstrapSlots": [c["slots"]]}
    # another slot count changes the hash: the pin is on the content
    ckks.dev_sidecar_write(path, rots, [c["slots"] // 2])
    assert hashlib.sha256(open(path, "rb").read()).hexdigest() != R17_DEV_SHA256


def test_empty_sidecar_of_the_default_keygen(ckks, tmp_path):
    """the client's default keygen writes writeDevSidecar(outDir, {}, {}) (mac_fhe_client.cpp:386)"""
    path = str(tmp_path / "d.dev")
    ckks.dev_sidecar_write(path, [], [])
    assert open(path, "rb").read() == (b"1 { 0 }\nAutoLoadCiphertexts: 1\nAutoLoadPlaintexts: 0\nRotationIndexes: { }\n"
                                       b"KeyDist: 1\nBootstrapSlots: { }\n")
    got = ckks.dev_sidecar_read(path)
    assert got["RotationIndexes"] == [] and got["BootstrapSlots"] == []


def test_reader_keeps_file_order_and_signs(ckks, tmp_path):
    path = str(tmp_path / "d.dev")
    with open(path, "w") as f:
        f.write("2 { 0 3 }\nAutoLoadCiphertexts: 0\nAutoLoadPlaintexts: 1\nRotationIndexes: { 5 -1 1024 -32768 }\n"
                "KeyDist: 2\nBootstrapSlots: { 32768 16 }\n")
    assert ckks.dev_sidecar_read(path) == {"devices": [0, 3], "AutoLoadCiphertexts": 0, "AutoLoadPlaintexts": 1,
                                           "KeyDist": 2, "RotationIndexes": [5, -1, 1024, -32768],
                                           "BootstrapSlots": [32768, 16]}


GOOD = ["1 { 0 }", "AutoLoadCiphertexts: 1", "AutoLoadPlaintexts: 0", "RotationIndexes: { 1 2 }", "KeyDist: 1",
        "BootstrapSlots: { 32768 }"]


def _variant(i, line):
    lines = list(GOOD)
    lines[i] = line
    return "\n".join(lines) + "\n"


MALFORMED = {
    "truncated": "\n".join(GOOD[:4]) + "\n",
    "no final newline": "\n".join(GOOD),
    "extra line": "\n".join(GOOD) + "\nKeyDist: 1\n",
    "swapped lines": "\n".join([GOOD[0], GOOD[2], GOOD[1]] + GOOD[3:]) + "\n",
    "device count": _variant(0, "2 { 0 }"),
    "device braces": _variant(0, "1 0"),
    "flag not integer": _variant(1, "AutoLoadCiphertexts: yes"),
    "flag key": _variant(2, "AutoLoadPlaintext: 0"),
    "rotation not integer": _variant(3, "RotationIndexes: { 1 x }"),
    "rotation brace": _variant(3, "RotationIndexes: { 1 2"),
    "rotation nested": _variant(3, "RotationIndexes: { 1 { 2 } }"),
    "rotation overflow": _variant(3, "RotationIndexes: { 99999999999 }"),
    "key dist missing value": _variant(4, "KeyDist:"),
    "slots not a power of two": _variant(5, "BootstrapSlots: { 3000 }"),
    "slots zero": _variant(5, "BootstrapSlots: { 0 }"),
    "slots key": _variant(5, "BootstrapSlot: { 32768 }"),
}


@pytest.mark.parametrize("name", sorted(MALFORMED))
def test_reader_refuses_malformed_files(ckks, tmp_path, name):
    path = str(tmp_path / "bad.dev")
    with open(path, "w") as f:
        f.write(MALFORMED[name])
    with pytest.raises(ckks.CkksError, match="dev sidecar"):
        ckks.dev_sidecar_read(path)


def test_good_variant_is_read(ckks, tmp_path):
    path = str(tmp_path / "good.dev")
    with open(path, "w") as f:
        f.write("\n".join(GOOD) + "\n")
    assert ckks.dev_sidecar_read(path)["RotationIndexes"] == [1, 2]


def _rot_index(k, N):
    """5^k mod 2N, negative k through the order N/2 of 5 (gpu_real_model.cu:1356-1360)"""
    return pow(5, k % (N // 2), 2 * N)


def _write_part(path, N, indices, seed_byte):
    """a part file of tiny keys (ring N) holding the given automorphism indices"""
    moduli = [97, 193, 257]                     # any layout: the resolver reads indices only
    records = [(g, bytes([seed_byte, i]) * 16, np.zeros((1, 3, N), dtype=np.uint64)) for i, g in enumerate(indices)]
    with open(path, "wb") as f:
        f.write(part_bytes(N, moduli, 2, 1, 1, 2, "tag", records))


def test_resolver_maps_each_rotation_to_its_key(ckks, tmp_path):
    """the automorphism index of rotation k is 5^k mod 2N (N of the parts); the first part holding it wins, in the
    order the parts are given; the sidecar's order is kept"""
    N = 64
    rots = [1, -1, 3, 5, -5, 2]
    g = {k: _rot_index(k, N) for k in rots}
    assert len(set(g.values())) == len(rots)
    p0, p1 = str(tmp_path / "evalrot.part000.seeded.bin"), str(tmp_path / "evalrot.part001.seeded.bin")
    _write_part(p0, N, [g[3], g[1], 7 if 7 not in g.values() else 9], 1)
    _write_part(p1, N, [g[-1], g[5], g[-5], g[2], g[1]], 2)
    dev = str(tmp_path / "cryptocontext.bin.dev")
    ckks.dev_sidecar_write(dev, rots, [N // 2])
    loc = ckks.rotation_keys_resolve(dev, [p0, p1])
    assert loc == [(0, 1, g[1]), (1, 0, g[-1]), (0, 0, g[3]), (1, 1, g[5]), (1, 2, g[-5]), (1, 3, g[2])]
    # a rotation by half the slots in either direction is one automorphism: both resolve to the same key
    ckks.dev_sidecar_write(dev, [N // 4, -(N // 4)], [])
    _write_part(p0, N, [_rot_index(N // 4, N)], 1)
    assert ckks.rotation_keys_resolve(dev, [p0]) == [(0, 0, _rot_index(N // 4, N))] * 2
    # the parts in the other order: rotation 1 now comes from the last record of the part listed first
    ckks.dev_sidecar_write(dev, rots, [N // 2])
    _write_part(p0, N, [g[3], g[1], 7 if 7 not in g.values() else 9], 1)
    loc2 = ckks.rotation_keys_resolve(dev, [p1, p0])
    assert loc2[0] == (0, 4, g[1])


def test_resolver_refuses_a_missing_key_and_mixed_rings(ckks, tmp_path):
    N = 64
    p0 = str(tmp_path / "p0.bin")
    _write_part(p0, N, [_rot_index(1, N)], 1)
    dev = str(tmp_path / "d.dev")
    ckks.dev_sidecar_write(dev, [1, 5], [])
    with pytest.raises(ckks.CkksError, match="no key for rotation 5"):
        ckks.rotation_keys_resolve(dev, [p0])
    p1 = str(tmp_path / "p1.bin")
    _write_part(p1, 2 * N, [_rot_index(5, 2 * N)], 2)
    with pytest.raises(ckks.CkksError, match="ring dimensions"):
        ckks.rotation_keys_resolve(dev, [p0, p1])


def test_contract_rotations_resolve_against_its_automorphism_indices(ckks, tmp_path):
    """every rotation amount of the r17 contract resolves, at N = 2^17, to one of the contract's automorphism indices
    (the index set its key parts were minted for, mac_fhe_client.cpp:418-440), through the engine's resolver.  The
    part file is sparse: a header, each record's index and seed, the b words left as holes (the resolver reads only
    the indices)."""
    import struct
    c = contract()
    N = c["ring"]
    rots = sorted(set(c["rotationAmounts"]))
    autos = sorted(set(c["autoIndices"]))
    head = part_bytes(N, [97], 1, 0, 1, 1, "tag", [], count=len(autos))
    rec = 4 + 32 + 8 * N
    p = str(tmp_path / "evalrot.part000.seeded.bin")
    with open(p, "wb") as f:
        f.write(head)
        for r, a in enumerate(autos):
            f.seek(len(head) + r * rec)
            f.write(struct.pack("<I", a) + bytes([r % 256]) * 32)
        f.truncate(len(head) + len(autos) * rec)
    dev = str(tmp_path / "cryptocontext.bin.dev")
    ckks.dev_sidecar_write(dev, rots, [c["slots"]])
    loc = ckks.rotation_keys_resolve(dev, [p])
    assert [g for (_, _, g) in loc] == [_rot_index(k, N) for k in rots]
    assert all(autos[r] == g for (_, r, g) in loc)
