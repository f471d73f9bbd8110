"""Writes synthetic_sha256.json: the SHA-256 of every tensor in synthetic.ENTRIES."""
import json
import os
import sys

sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))
import synthetic  # noqa: E402

if __name__ == "__main__":
    out = {name: synthetic.digest(gen()) for name, (gen, _) in synthetic.ENTRIES.items()}
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "synthetic_sha256.json")
    with open(path, "w") as f:
        json.dump(out, f, indent=1, sort_keys=True)
        f.write("\n")
    print(f"{len(out)} digests -> {path}")
