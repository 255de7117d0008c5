"""CPU tests of the on-disk format loaders (libpih_amd_artifacts.so) and of
the test writer that feeds them:

* the writer's metadata region equals the reference serialiser's, byte for
  byte (golden vectors from QwenInt4ArtifactMetadata::serialize_fixed_region);
* the library's official layout equals the writer's, record by record, and
  its totals are the reference's constants (qwen3_int4_artifact_layout.h:33-39);
* a whole canonical file (539,758,592 bytes, written sparse) verifies, and
  each corruption the reference's loader rejects is rejected with the same
  status class; the live reference parser agrees where oracle/_ref is built;
* the DeepSeek expert bundle bind reproduces the reference's known answers
  (tests/cpp/model/deepseek_expert_bundle_layout_test.cpp:10-43).
"""
import hashlib
import mmap
import os
import struct

import numpy as np
import pytest

import oracle
from pih_amd import abi, artifacts
from tests import artifact_files as af

GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "ref_vectors.npz")


def test_metadata_writer_matches_reference_serializer():
    gold = np.load(GOLDEN, allow_pickle=False)["qwen_meta_region"].tobytes()
    roots, digests = af.golden_roots_and_digests()
    region = af.qwen_metadata(roots, digests)
    assert region[:len(gold)] == gold
    assert region[len(gold):] == bytes(len(region) - len(gold))


def test_library_layout_matches_reference_layout():
    layout = af.qwen_layout()
    assert len(layout) == artifacts.RECORD_COUNT
    kinds = {k: sum(r[1] == k for r in layout) for k in range(1, 6)}
    assert kinds == {1: 196, 2: 196, 3: 1, 4: 113, 5: 1}
    assert sum(r[4] for r in layout) == 538_378_240
    for ident, kind, _, _, logical, offset, extent, rows, cols in layout:
        r = artifacts.qwen_int4_record(ident)
        assert (r.kind, r.logical_bytes, r.file_offset, r.extent_bytes, r.rows, r.columns) == (
            kind, logical, offset, extent, rows, cols), ident
    head = artifacts.qwen_int4_record("lm_head.weight")
    emb = artifacts.qwen_int4_record("model.embed_tokens.weight")
    assert head.kind == artifacts.ALIAS and head.device_offset == emb.device_offset == emb.file_offset - (1 << 20)
    with pytest.raises(artifacts.ArtifactError):
        artifacts.qwen_int4_record("model.layers.28.mlp.up_proj.weight.scales")


@pytest.fixture(scope="module")
def canonical_file(tmp_path_factory):
    path = str(tmp_path_factory.mktemp("qwen") / "qwen3-0.6b-int4.xing")
    payloads = {}
    for seed, src in ((1, "model.layers.0.mlp.gate_proj.weight"), (2, "model.layers.27.self_attn.o_proj.weight")):
        n, k = (3072, 1024) if "gate" in src else (1024, 2048)
        packed, scales = af.int4_linear_payloads(seed, src, n, k)
        payloads[src + ".packed_values"], payloads[src + ".scales"] = packed, scales
    payloads["model.norm.weight"] = np.arange(1024, dtype=np.uint16).tobytes()
    af.write_qwen_artifact(path, payloads)
    return path


def _status(fn):
    try:
        fn()
    except artifacts.ArtifactError as e:
        return e.status.code
    return abi.OK


def test_canonical_file_verifies(canonical_file):
    with open(canonical_file, "r+b") as f:
        mm = mmap.mmap(f.fileno(), 0)
        info = artifacts.verify_qwen_int4(mm, payloads=True)
        assert (info.record_count, info.payload_record_count, info.file_bytes, info.padded_data_bytes) == (
            507, 506, af.FILE_BYTES, artifacts.DATA_BYTES)
        assert bytes(info.source_artifact_root) == af.golden_roots_and_digests()[0][:32]
        mm.close()


def _reseal(mm):
    """Recomputes the metadata checksum after an edit of the region."""
    enc = struct.unpack_from("<I", mm, 12)[0]
    body = bytearray(mm[:enc])
    body[120:152] = bytes(32)
    mm[120:152] = hashlib.sha256(bytes(body)).digest()


def test_corruptions_are_rejected(canonical_file):
    R = oracle.ref()
    gate = artifacts.qwen_int4_record("model.layers.0.mlp.gate_proj.weight.packed_values")
    norm = artifacts.qwen_int4_record("model.norm.weight")
    with open(canonical_file, "r+b") as f:
        mm = mmap.mmap(f.fileno(), 0)

        def check(edit, want, region_only=False):
            saved = bytes(mm[:1 << 20]), bytes(mm[gate.file_offset:gate.file_offset + 16]), \
                bytes(mm[norm.file_offset + norm.logical_bytes:norm.file_offset + norm.logical_bytes + 4])
            edit()
            try:
                assert _status(lambda: artifacts.verify_qwen_int4(mm, payloads=True)) == want
                if region_only and R is not None:
                    region = np.frombuffer(mm, np.uint8, count=1 << 20).copy()
                    assert (R.pr_qwen_int4_parse(region.ctypes.data_as(oracle.P)) == 0) == (want == abi.OK)
            finally:
                mm[:1 << 20] = saved[0]
                mm[gate.file_offset:gate.file_offset + 16] = saved[1]
                mm[norm.file_offset + norm.logical_bytes:norm.file_offset + norm.logical_bytes + 4] = saved[2]

        def setb(at, value):
            def f():
                mm[at] = value
            return f

        check(lambda: None, abi.OK, region_only=True)
        # payload byte changed: digest mismatch
        check(setb(gate.file_offset + 3, mm[gate.file_offset + 3] ^ 0x10), abi.FAILED_PRECONDITION)
        # non-zero padding after a payload
        check(setb(norm.file_offset + norm.logical_bytes + 1, 1), abi.FAILED_PRECONDITION)
        # metadata byte changed without resealing: checksum mismatch
        check(setb(400, mm[400] ^ 1), abi.FAILED_PRECONDITION, region_only=True)
        # bad magic, version, record count, reserved field: header errors
        check(setb(0, ord("Y")), abi.INVALID_ARGUMENT, region_only=True)
        for at, val in ((8, 2), (16, 0), (20, 1)):
            check(lambda at=at, val=val: (mm.__setitem__(at, val), _reseal(mm)), abi.INVALID_ARGUMENT,
                  region_only=True)
        # non-zero byte in the tail after the encoded metadata
        check(setb((1 << 20) - 1, 7), abi.INVALID_ARGUMENT, region_only=True)
        # a record's offset changed (resealed): record mismatch
        enc_first = 160 + len(af.FORMAT_ID) + len(af.LAYOUT_ID)
        check(lambda: (mm.__setitem__(slice(enc_first + 16, enc_first + 17), bytes([mm[enc_first + 16] ^ 0x10])),
                       _reseal(mm)), abi.FAILED_PRECONDITION, region_only=True)
        # format identifier changed (resealed)
        check(lambda: (mm.__setitem__(160, ord("y")), _reseal(mm)), abi.INVALID_ARGUMENT, region_only=True)
        # empty root (resealed)
        check(lambda: (mm.__setitem__(slice(56, 88), bytes(32)), _reseal(mm)), abi.FAILED_PRECONDITION,
              region_only=True)
        # metadata-only verification skips payload digests
        mm[gate.file_offset + 5] ^= 0x01
        try:
            assert _status(lambda: artifacts.verify_qwen_int4(mm, payloads=False)) == abi.OK
        finally:
            mm[gate.file_offset + 5] ^= 0x01
        # a file of the wrong length
        assert _status(lambda: artifacts.verify_qwen_int4(bytearray(mm[:1 << 20]), payloads=False)) == \
            abi.FAILED_PRECONDITION
        mm.close()


def test_expert_bundle_bind_reference_kats():
    v = artifacts.bind_expert_bundle(0x10000000)
    assert (v.w1_packed, v.w1_scales, v.w2_packed, v.w2_scales, v.w3_packed, v.w3_scales) == (
        0x10000000, 0x10400000, 0x10440000, 0x10840000, 0x10880000, 0x10C80000)
    assert (v.packed_bytes, v.scale_bytes) == (4194304, 262144)
    assert v.w3_scales + v.scale_bytes == 0x10000000 + artifacts.BUNDLE_BYTES
    for bad in (0, 0x10000001, (2 ** 64 - 256) & ~255):
        with pytest.raises(artifacts.ArtifactError):
            artifacts.bind_expert_bundle(bad)
