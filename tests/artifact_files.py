"""Test infrastructure: writers of the on-disk weight formats, restated from
the reference so the loaders in libpih_amd_artifacts.so can be fed canonical
files.  The metadata serialiser is pinned byte for byte to the reference's
own (tests/golden/ref_vectors.npz, made by QwenInt4ArtifactMetadata::
serialize_fixed_region compiled from the reference sources).

  qwen_layout()        the official record list: 28 layers x 7 projections
                       (packed values [N][K/2] + fp16 scales [N][K/128]),
                       113 bf16 norms, the bf16 embedding and the tied
                       lm_head alias, sorted by identity, payload extents
                       4096-aligned from 1 MiB
                       (qwen3_int4_artifact_layout.cpp:41-104,
                       qwen3_int4_linear_shape_ledger.cpp:14-31,72-110)
  qwen_metadata()      the 1 MiB metadata region
                       (qwen3_int4_artifact_metadata.cpp:113-143)
  write_qwen_artifact  a whole canonical file with chosen payloads (the
                       rest zero), digests over the payload bytes
"""
import hashlib
import struct

import numpy as np

META = 1 << 20
FILE_BYTES = 539_758_592
FORMAT_ID = b"xing-w4a16-sym-g128-v1"
LAYOUT_ID = b"canonical-nk-low-nibble-k-v1"
PROJECTIONS = (("self_attn.q_proj.weight", 2048, 1024), ("self_attn.k_proj.weight", 1024, 1024),
               ("self_attn.v_proj.weight", 1024, 1024), ("self_attn.o_proj.weight", 1024, 2048),
               ("mlp.gate_proj.weight", 3072, 1024), ("mlp.up_proj.weight", 3072, 1024),
               ("mlp.down_proj.weight", 1024, 3072))
NORMS = (("input_layernorm.weight", 1024), ("post_attention_layernorm.weight", 1024),
         ("self_attn.q_norm.weight", 128), ("self_attn.k_norm.weight", 128))


def qwen_layout():
    """[(identity, kind, source, alias, logical, offset, extent, rows, cols)]"""
    recs = [("model.embed_tokens.weight", 3, "model.embed_tokens.weight", "", 151936 * 1024 * 2, 151936, 1024),
            ("lm_head.weight", 5, "lm_head.weight", "model.embed_tokens.weight", 0, 151936, 1024)]
    for layer in range(28):
        pre = f"model.layers.{layer}."
        for suffix, n, k in PROJECTIONS:
            src = pre + suffix
            recs.append((src + ".packed_values", 1, src, "", n * k // 2, n, k))
            recs.append((src + ".scales", 2, src, "", n * (k // 128) * 2, n, k))
        for name, width in NORMS:
            recs.append((pre + name, 4, pre + name, "", width * 2, 1, width))
    recs.append(("model.norm.weight", 4, "model.norm.weight", "", 2048, 1, 1024))
    recs.sort(key=lambda r: r[0].encode())
    out, offset = [], META
    for ident, kind, src, alias, logical, rows, cols in recs:
        if kind == 5:
            out.append((ident, kind, src, alias, 0, 0, 0, rows, cols))
            continue
        extent = -(-logical // 4096) * 4096
        out.append((ident, kind, src, alias, logical, offset, extent, rows, cols))
        offset += extent
    assert len(out) == 507 and offset == FILE_BYTES
    return out


def qwen_metadata(roots: bytes, digests) -> bytes:
    """The 1 MiB region for three 32-byte roots and one digest per payload
    record (layout order, aliases skipped)."""
    layout = qwen_layout()
    digests = list(digests)
    body = bytearray()
    body += b"XINGW4A1" + struct.pack("<IIII", 1, 0, len(layout), 0) + roots + bytes(32)
    body += struct.pack("<HHI", len(FORMAT_ID), len(LAYOUT_ID), 0) + FORMAT_ID + LAYOUT_ID
    di = 0
    for ident, kind, src, alias, logical, offset, extent, _, _ in layout:
        if kind == 5:
            dig = bytes(32)
        else:
            dig = digests[di]
            di += 1
        body += struct.pack("<BBHHHQQQ", kind, 0, len(ident), len(src), len(alias), logical, offset, extent)
        body += dig + ident.encode() + src.encode() + alias.encode()
    assert di == len(digests) == 506
    body[12:16] = struct.pack("<I", len(body))
    body[120:152] = hashlib.sha256(bytes(body)).digest()
    return bytes(body) + bytes(META - len(body))


def golden_roots_and_digests():
    roots = b"".join(hashlib.sha256(b"pih-golden-root-%d" % i).digest() for i in range(3))
    digests = [hashlib.sha256(b"pih-golden-payload-%d" % i).digest() for i in range(506)]
    return roots, digests


def write_qwen_artifact(path, payloads: dict, roots: bytes = None):
    """Writes a canonical file: ``payloads`` maps identity -> bytes (exactly
    that record's logical size); every other payload is zero."""
    layout = qwen_layout()
    roots = roots or golden_roots_and_digests()[0]
    digests = []
    with open(path, "wb") as f:
        f.truncate(FILE_BYTES)
        for ident, kind, _, _, logical, offset, _, _, _ in layout:
            if kind == 5:
                continue
            data = payloads.get(ident)
            if data is not None:
                assert len(data) == logical, ident
                f.seek(offset)
                f.write(data)
                digests.append(hashlib.sha256(data).digest())
            else:
                digests.append(_zero_digest(logical))
        f.seek(0)
        f.write(qwen_metadata(roots, digests))
    return layout


_ZERO = {}


def _zero_digest(n: int) -> bytes:
    if n not in _ZERO:
        h = hashlib.sha256()
        chunk = bytes(min(n, 1 << 22))
        left = n
        while left:
            take = min(left, len(chunk))
            h.update(chunk[:take])
            left -= take
        _ZERO[n] = h.digest()
    return _ZERO[n]


def int4_linear_payloads(seed: int, source: str, n: int, k: int):
    """Random symmetric INT4 codes in [-7, 7] (low nibble = even k) and fp16
    scales in [0.001, 0.02]: (packed bytes, scale bytes)."""
    rng = np.random.default_rng(seed)
    q = rng.integers(-7, 8, size=(n, k)).astype(np.int8)
    nib = (q & 0x0F).astype(np.uint8)
    packed = (nib[:, 0::2] | (nib[:, 1::2] << 4)).astype(np.uint8)
    scales = rng.uniform(0.001, 0.02, size=(n, k // 128)).astype(np.float16)
    return packed.tobytes(), scales.tobytes()
