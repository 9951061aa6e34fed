"""Write the trained-encoder fixture `qwen3_8b_encoders.npz` from the
reference's Qwen3-8B encoder bundle (pretrained/Qwen3-8B: 288 tensor-only
`lLL_gGG.pt` files plus manifest.json, pretrained/README.md:9-13).

The bundle is read through `prismkv_amd.weights.load_encoders`, which checks
every file's sha256 against the manifest and loads tensors only
(`torch.load(weights_only=True)`), the checks of src/prismkv/weights.py:41-70.
Four units are kept, chosen to span the bundle: the first unit, the units
with the smallest and the largest saved key scale, and the last unit.  For
each the fixture holds W_enc f32 [3000,128], b_enc f32 [3000], the saved
key and query scales, key_mean, query_topk, the unit's (layer, group) and the
sha256 and name of its source file, so a test can tie the fixture back to the bundle.

Run in a container that holds the reference (the GPU tests only read the
fixture):

    python tests/golden/make_trained_encoders.py [/root/reference/pretrained/Qwen3-8B]
"""
import sys
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT))

from prismkv_amd.weights import load_encoders  # noqa: E402

BUNDLE = Path("/root/reference/pretrained/Qwen3-8B")
OUT = Path(__file__).with_name("qwen3_8b_encoders.npz")


def pick_units(manifest):
    rows = manifest["groups"]
    by_scale = sorted(rows, key=lambda r: r["key_scale"])
    picks = [rows[0], by_scale[0], by_scale[-1], rows[-1]]
    units = []
    for r in picks:
        unit = (r["layer"], r["group"])
        if unit not in units:
            units.append(unit)
    return units


def main(bundle=BUNDLE, out=OUT):
    encoders, manifest = load_encoders(bundle)
    assert len(encoders) == 288, len(encoders)
    units = pick_units(manifest)
    rows = {(r["layer"], r["group"]): r for r in manifest["groups"]}
    W = np.stack([encoders[u].sae.W_enc.detach().numpy() for u in units]).astype(np.float32)
    b = np.stack([encoders[u].sae.b_enc.detach().numpy() for u in units]).astype(np.float32)
    np.savez_compressed(
        out,
        W_enc=W,
        b_enc=b,
        key_scale=np.array([encoders[u].key_scale for u in units], np.float64),
        query_scale=np.array([encoders[u].query_scale for u in units], np.float64),
        key_mean=np.array([rows[u]["key_mean"] for u in units], np.int64),
        query_topk=np.array([rows[u]["query_topk"] for u in units], np.int64),
        layer=np.array([u[0] for u in units], np.int64),
        group=np.array([u[1] for u in units], np.int64),
        sha256=np.array([rows[u]["sha256"] for u in units], dtype="<U64"),
        unit_file=np.array([rows[u]["file"] for u in units], dtype="<U16"),
    )
    print(f"wrote {out} ({out.stat().st_size / 1e6:.2f} MB): units {units}")


if __name__ == "__main__":
    main(Path(sys.argv[1]) if len(sys.argv) > 1 else BUNDLE)
