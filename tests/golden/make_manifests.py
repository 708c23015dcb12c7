"""Writes tests/golden/manifests.json from the reference's committed model
manifests (runtime/model-artifacts/*/manifest.json): for each, the model id
and the commitments it must be the hash of (direct.rs:96-105), the family,
the names of its shape fields and its version. Data only; run in the
container that holds the reference."""
import glob
import json
import os

REF = "/root/reference/runtime/model-artifacts"
OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "manifests.json")

out = {}
for path in sorted(glob.glob(os.path.join(REF, "*", "manifest.json"))):
    with open(path) as f:
        m = json.load(f)
    out[os.path.basename(os.path.dirname(path))] = {
        "version": m["version"], "family": m.get("family"), "model_id": m.get("model_id"),
        "model_commitments": m.get("model_commitments"), "shape_fields": sorted(m["shape"]),
    }
with open(OUT, "w") as f:
    json.dump({"source": "runtime/model-artifacts/*/manifest.json", "manifests": out}, f, indent=1)
print(f"{len(out)} manifests -> {OUT}")
