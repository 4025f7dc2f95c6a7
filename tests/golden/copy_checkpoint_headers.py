"""Copy the reference's real-checkpoint metadata fixtures.

packages/hf_config/testdata/<name>/ of the reference holds, for 13 published
checkpoints, config.json, the exact header bytes of each safetensors shard
(the 8-byte length prefix and the JSON header, no weight data), the sharded
index, the shard file sizes (sizes.json) and the revision they came from
(provenance.json). This copies those data files unchanged into
tests/golden/checkpoints/<name>/. Run in a container where the reference is
mounted:

    python tests/golden/copy_checkpoint_headers.py /root/reference
"""
import os
import shutil
import sys

KEEP = ("config.json", "model.safetensors.index.json", "sizes.json", "provenance.json")


def main(ref_root: str) -> None:
    src = os.path.join(ref_root, "packages", "hf_config", "testdata")
    dst = os.path.join(os.path.dirname(os.path.abspath(__file__)), "checkpoints")
    total = 0
    for name in sorted(os.listdir(src)):
        if not os.path.isdir(os.path.join(src, name)):
            continue
        os.makedirs(os.path.join(dst, name), exist_ok=True)
        for f in sorted(os.listdir(os.path.join(src, name))):
            if f in KEEP or f.endswith(".safetensors.header"):
                shutil.copyfile(os.path.join(src, name, f), os.path.join(dst, name, f))
                total += os.path.getsize(os.path.join(dst, name, f))
    print(f"copied {total} bytes into {dst}")


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
