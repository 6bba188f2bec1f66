"""Descriptor front end on the GPU: the ROM the reference's generator built
for the pruned synthetic model (tests/golden/e2e_rom.mem) and its weight
region (pinned against the reference's serialize_weights in
tests/test_schedule_cpu.py), run over the 32 pruned images and compared with
the reference golden model's checkpoints; then a whole e2e vector directory
through heatvit_amd.schedule.run_vectors."""

from pathlib import Path

import numpy as np
import pytest

import golden_io as gio
import memory_image as mi
from heatvit_amd import synth

pytestmark = pytest.mark.gpu
ROM = Path(__file__).resolve().parent / "golden" / "e2e_rom.mem"


def _region():
    from heatvit_amd.schedule import compile_rom, read_rom
    words = read_rom(ROM)
    return words, mi.weight_region(synth.pruned_params(), compile_rom(words))


def test_rom_forward_matches_the_golden_checkpoints():
    from heatvit_amd.schedule import run
    meta, arrays = gio.load("pruned")
    imgs, _ = synth.pruned_workload()
    words, region = _region()
    logits, cks, counts = run(words, region, imgs)
    for i in range(len(imgs)):
        assert np.array_equal(logits[i], arrays["logits"][i]), i
        got = {name: np.frombuffer(v[i], np.int8) for name, v in cks.items() if v[i]}
        got["logits"] = logits[i]
        digests = gio.model_checkpoint_digests(got)
        bad = [k for k, v in meta["checkpoints"][i].items() if digests.get(k) != v]
        assert not bad, (i, bad)
        rows = meta["rows"][i]
        assert counts[i].tolist() == [rows["block_01"], rows["block_04"], rows["block_07"],
                                      rows["block_10"]]


def test_vector_directory(tmp_path, oracle):
    from heatvit_amd.schedule import run_vectors
    imgs, params = synth.pruned_workload(1)
    _, region = _region()
    logits, cks, _, _ = oracle.model_infer(imgs[0], params)
    d = mi.vector_dir(tmp_path / "e2e", imgs[0], region,
                      {k: np.ascontiguousarray(v, np.int8).tobytes() for k, v in cks.items()
                       if k != "logits"}, logits)
    result = run_vectors(d, ROM)
    assert len(result) == 18 and all(result.values()), result
