"""Writes the descriptor front end's fixtures by running the reference's
schedule and memory-image generators (tools/generate_descriptors.py,
tools/generate_e2e_vectors.py) in the development container:

  tests/golden/e2e_rom.mem      build_schedule(build_memory_map(), table) for
                                this build's pruned synthetic model (its
                                per-tensor exponents as a scale table),
                                format_desc_hex lines;
  tests/golden/e2e_errors/*.mem write_error_roms (the engine's error and
                                warning injection ROMs);
  tests/golden/e2e.json         the weight map, the SHA-256 of
                                serialize_weights(...) for the same model,
                                the checkpoint layout for the first pruned
                                images' token counts, and the weight map of
                                the reference's committed synthetic ROM.

Run:  python tests/golden/make_e2e.py
"""

import hashlib
import json
import os
import shutil
import sys
import tempfile
from pathlib import Path

ROOT = Path(__file__).resolve().parents[2]
REFERENCE = Path(os.environ.get("HEATVIT_REFERENCE", "/root/reference"))
OUT = Path(__file__).resolve().parent
sys.path[:0] = [str(ROOT), str(OUT)]

from heatvit_amd import synth  # noqa: E402
from heatvit_amd.scale_table import ScaleTable  # noqa: E402


def main():
    sys.path.insert(0, str(REFERENCE))
    import make_golden
    from tools import generate_descriptors as gd
    from tools import generate_e2e_vectors as ge
    from tools.p2.scale_table import ScaleTable as RefTable
    from verification.heatvit_ref.descriptor import format_desc_hex

    params = synth.pruned_params()
    table = ScaleTable.from_params(params).validate()
    mm, scratch_bytes, weight_bytes = gd.build_memory_map()
    descs = gd.build_schedule(mm, RefTable(table.weights, table.activations).validate())
    (OUT / "e2e_rom.mem").write_text("".join(format_desc_hex(d.pack()) + "\n" for d in descs))

    weights = ge.serialize_weights(make_golden.ref_model(params), mm["weight"])
    meta = json.loads((OUT / "pruned.json").read_text())
    layouts = []
    for rows in meta["rows"][:4]:
        counts = [rows["block_01"], rows["block_04"], rows["block_07"], rows["block_10"]]
        layout = ge.checkpoint_layout(mm, counts)
        layouts.append({"token_counts": counts,
                        "checkpoints": {k: {"region": v[0], "offset": v[1], "bytes": v[2],
                                            "desc_index": v[4]} for k, v in layout.items()}})
    fixture = {
        "weight_map": mm["weight"], "weight_bytes": weight_bytes, "scratch_bytes": scratch_bytes,
        "weights_sha256": hashlib.sha256(weights).hexdigest(), "weights_len": len(weights),
        "layouts": layouts,
        "committed_rom_sha256": hashlib.sha256(
            (REFERENCE / "rtl/generated/heatvit_descriptors.mem").read_bytes()).hexdigest(),
    }
    (OUT / "e2e.json").write_text(json.dumps(fixture, indent=1) + "\n")

    errs = OUT / "e2e_errors"
    errs.mkdir(exist_ok=True)
    with tempfile.TemporaryDirectory() as tmp:
        ge.write_error_roms(tmp)
        for f in sorted(Path(tmp, "errors").glob("*.mem")):
            shutil.copy(f, errs / f.name)
    print(f"wrote {len(descs)} descriptors, weights {len(weights)} B, "
          f"{len(list(errs.glob('*.mem')))} error ROMs")


if __name__ == "__main__":
    main()
