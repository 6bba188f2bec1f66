"""GPU counterparts of the engine's error and warning cases
(sim/tb/tb_heatvit_errors.sv cases 4 and 8-10, heatvit_pkg.sv:109-122):
per-image warning bits of the HIP forward against the oracle's, per-image
token-count status of the block, and the error code carried by the Python
exceptions."""

import numpy as np
import pytest
import torch

import warning_cases as wc
from heatvit_amd import _lib, synth

pytestmark = pytest.mark.gpu


def test_model_warning_bits_vs_oracle(oracle):
    from heatvit_amd.model import HeatViTModel
    imgs, params = synth.pruned_workload(4)
    cases = {
        "ln_negative_variance": wc.ln_negative_variance_model(synth.unpruned_control(params)),
        "head_den_zero": wc.with_selector(params, 0, wc.head_den_zero_selector),
        "package_den_zero": wc.with_selector(params, 2, wc.package_den_zero_selector),
        "head_and_package": wc.with_selector(
            wc.with_selector(params, 2, wc.package_den_zero_selector), 1,
            wc.head_den_zero_selector),
        "none": params,
    }
    seen = set()
    for name, p in cases.items():
        print(f"model warnings case {name}", flush=True)
        r = HeatViTModel().infer_batch(imgs, p)
        logits, counts, status, warnings = oracle.model_infer_batch(imgs, p, threads=4)
        assert not status.any()
        assert np.array_equal(r.logits, logits), name
        assert np.array_equal(r.token_counts, counts), name
        assert np.array_equal(r.warnings, warnings), (name, r.warnings, warnings)
        seen |= set(warnings.tolist())
    assert seen == {0, 1, 2, 3, 4}
    one = HeatViTModel().infer(imgs[0], cases["head_and_package"])
    assert one.warnings == 3


def test_block_ln_warning_per_image(oracle):
    from heatvit_amd.transformer import transformer_block_batch
    _, bp = synth.block_workload()
    bp = wc.ln_negative_variance_block(bp)
    rng = np.random.default_rng(11)
    lens = [197, 40, 3, 120, 1, 66]
    xs = [rng.integers(-40, 41, (n, 192)).astype(np.int8) for n in lens]
    for i, row in ((0, 5), (3, 119), (4, 0)):
        xs[i][row] = wc.LN_NEG_ROW
    zs, warn = transformer_block_batch(xs, bp, warnings=True)
    want = []
    for i, xi in enumerate(xs):
        z, ck = oracle.transformer_block(xi, bp, checkpoints=False)
        assert np.array_equal(zs[i], z), i
        want.append(ck["warnings"])
    assert warn.tolist() == want
    assert want[0] == want[3] == want[4] == _lib.HV_WARN_LN_NEGATIVE_VARIANCE
    assert 0 in want


def _block_call(dev, x, offsets, max_rows, status, warn, ws, z):
    L = _lib.lib()
    return L.hv_block_forward(dev.struct, x.data_ptr(), offsets.data_ptr(), len(offsets) - 1,
                              max_rows, z.data_ptr(), None, status.data_ptr(), warn.data_ptr(),
                              ws.data_ptr(), ws.numel(), torch.cuda.current_stream().cuda_stream)


def test_block_token_count_status(oracle):
    """Images whose row count leaves [1, 197] or whose rows leave the
    buffers get HV_ERR_TOKEN_COUNT and are skipped by the attention; the
    valid images of the same call are still exact."""
    from heatvit_amd.device import DeviceBlock
    _, bp = synth.block_workload()
    dev = DeviceBlock(bp)
    rng = np.random.default_rng(5)
    cap = 400
    xh = rng.integers(-128, 128, (cap, 192)).astype(np.int8)
    x = torch.from_numpy(xh).cuda()
    z = torch.zeros((cap, 192), dtype=torch.int8, device="cuda")
    L = _lib.lib()
    # Image b owns rows offsets[b] .. offsets[b+1]:
    #   0 [0, 50) ok      1 [50, 50) empty       2 [50, 80) ok
    #   3 [80, 278) 198 rows                      4 [278, 280) ok
    #   5 [280, 100) negative count               6 [100, 160) ok
    #   7 [160, 360) 200 rows                     8 [360, 410) past the 400 rows
    # The valid images' rows do not overlap; the GEMMs and LayerNorms run on
    # min(offsets[B], 400) rows, all inside the buffers.
    offsets = [0, 50, 50, 80, 278, 280, 100, 160, 360, 410]
    batch = len(offsets) - 1
    ws = torch.empty(L.hv_block_workspace_bytes(batch, cap), dtype=torch.uint8, device="cuda")
    status = torch.full((batch,), -1, dtype=torch.int32, device="cuda")
    warn = torch.full((batch,), -1, dtype=torch.int32, device="cuda")
    print("block status case offsets", offsets, flush=True)
    off = torch.tensor(offsets, dtype=torch.int32, device="cuda")
    _lib.check(_block_call(dev, x, off, cap, status, warn, ws, z), "block")
    torch.cuda.synchronize()
    tc = _lib.HV_ERR_TOKEN_COUNT
    assert status.cpu().tolist() == [0, tc, 0, tc, 0, tc, 0, tc, tc]
    zh, wh = z.cpu().numpy(), warn.cpu().numpy()
    for b in (0, 2, 4, 6):
        lo, hi = offsets[b], offsets[b + 1]
        ref, ck = oracle.transformer_block(xh[lo:hi], bp, checkpoints=False)
        assert np.array_equal(zh[lo:hi], ref), b
        assert wh[b] == ck["warnings"] == 0, b


def test_python_errors_carry_the_engine_code():
    from heatvit_amd.model import Engine
    from heatvit_amd.transformer import transformer_block_batch
    _, params = synth.pruned_workload(1)
    eng = Engine(params, 2)
    eng.workspace = eng.workspace[:1024]
    images = torch.zeros((2, 224 * 224 * 3), dtype=torch.int8, device="cuda")
    with pytest.raises(ValueError) as e:
        eng.forward(images)
    assert e.value.error_class == _lib.HV_ERR_ADDRESS
    x, bp = synth.block_workload()
    with pytest.raises(ValueError):
        transformer_block_batch([x[:0]], bp)  # host check: 1..197 rows per image
