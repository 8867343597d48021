"""Writes envelope_keys.json: the key structure (names only, no values) of the reference's
committed benchmark artefacts bench/results/gpu.json (the GPU example's envelope,
crates/core/examples/gpu_knn.rs:274-333) and bench/results/sift1m.json (the harness
envelope, bench/harness.py:157-198). tests/test_envelope.py checks this backend's envelopes
against it. Run from the repository root with the reference at /root/reference."""
import json
from pathlib import Path

REF = Path("/root/reference/bench/results")


def keys(obj):
    if isinstance(obj, dict):
        return {k: keys(v) for k, v in obj.items()}
    if isinstance(obj, list) and obj and isinstance(obj[0], dict):
        return [keys(obj[0])]
    return None


out = {name: keys(json.loads((REF / f"{name}.json").read_text())) for name in ("gpu", "sift1m")}
dst = Path(__file__).resolve().parent / "envelope_keys.json"
dst.write_text(json.dumps(out, indent=1, sort_keys=True) + "\n")
print(f"wrote {dst}")
