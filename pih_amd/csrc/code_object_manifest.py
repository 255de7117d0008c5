"""Write the JSON manifest that travels beside a gfx950 code object.

The Qwen model checks its device image against a small manifest before
loading it (the reference's pih.cubin_artifact.v1: schema, target_sm,
producer_toolkit, producer_flags_sha256, cubin_sha256, cubin_bytes;
src/backend/cuda/cubin_artifact_manifest.cpp:12-91).  The gfx950 manifest
keeps the same six fields under code-object names:

  {"schema": "pih.code_object_artifact.v1", "target": "gfx950",
   "producer_toolchain": "<hipcc version line>",
   "producer_flags_sha256": "<sha256 of the compile flags>",
   "code_object_sha256": "<sha256 of the .hsaco>", "code_object_bytes": N}

usage: code_object_manifest.py <hsaco> <target> <toolchain> <flags...>
"""
import hashlib
import json
import os
import sys


def main(argv):
    if len(argv) < 4:
        print(__doc__, file=sys.stderr)
        return 2
    path, target, toolchain = argv[1], argv[2], argv[3]
    flags = " ".join(argv[4:])
    data = open(path, "rb").read()
    if len(data) < 64 or data[:4] != b"\x7fELF":
        print(f"{path}: not an ELF code object", file=sys.stderr)
        return 1
    manifest = {
        "schema": "pih.code_object_artifact.v1",
        "target": target,
        "producer_toolchain": toolchain[:128],
        "producer_flags_sha256": hashlib.sha256(flags.encode()).hexdigest(),
        "code_object_sha256": hashlib.sha256(data).hexdigest(),
        "code_object_bytes": len(data),
    }
    out = path + ".json"
    with open(out + ".tmp", "w") as f:
        json.dump(manifest, f, sort_keys=True)
        f.write("\n")
    os.replace(out + ".tmp", out)
    return 0


if __name__ == "__main__":
    sys.exit(main(sys.argv))
