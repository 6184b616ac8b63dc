"""jq_history_reconstruct_noalloc through the C ABI on an MI355X: the same rows
as jq_history_reconstruct (observations in f32 and u8 + aux, globals, packed
and bool canonical masks), bit for bit, on two calls in a row, the second with
a smaller batch; device memory does not move across any of the calls, the
first included; a batch above the maximum is refused."""

from __future__ import annotations

import numpy as np
import pytest

torch = pytest.importorskip("torch")

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def jq():
    if not torch.cuda.is_available():
        pytest.fail("GPU test collected on a machine without a visible GPU")
    import junqi_amd
    return junqi_amd


def _outputs(dev, batch, fmt):
    dt = {"f32": torch.float32, "u8": torch.uint8}[fmt]
    return {"spatial": torch.full((batch, 317, 17, 17), 7, dtype=dt, device=dev),
            "aux": torch.full((batch, 2320), 7, dtype=torch.uint8, device=dev) if fmt == "u8" else None,
            "global": torch.full((batch, 28), 7, dtype=torch.float32, device=dev),
            "mask_words": torch.full((batch, 521), 7, dtype=torch.int32, device=dev),
            "mask_bool": torch.full((batch, 16641), 7, dtype=torch.uint8, device=dev)}


def _call(jq, fn, hist, flat, obs, fmt, out):
    from junqi_amd import _lib as L
    P = lambda t: None if t is None else t.data_ptr()  # noqa: E731
    code = {"f32": L.OBS_F32, "u8": L.OBS_U8}[fmt]
    rc = fn(hist._h, flat.data_ptr(), obs.data_ptr(), int(flat.numel()), code, P(out["spatial"]), P(out["aux"]),
            P(out["global"]), P(out["mask_words"]), P(out["mask_bool"]),
            torch.cuda.current_stream().cuda_stream)
    L.check(rc)


def test_noalloc_reconstruct_equals_reconstruct(jq):
    from junqi_amd import _lib as L
    n, steps, show = 256, 6, 1
    print(f"[noalloc] n={n} steps={steps}", flush=True)
    ro = jq.GpuRollout(n, show_mode=show, max_num_moves=400)
    ro.reset(17)
    hist = ro.create_rollout_history(steps)
    dev = ro.device
    rng = np.random.default_rng(3)
    for t in range(steps):
        hist.snapshot(ro.state, ro.turn_torch().clone(), t)
        b = ro.state
        b.legal()
        acts = b.sample_uniform(5, t)
        b.step(acts)
    torch.cuda.synchronize()
    rows = steps * n
    for batch, fmt in ((900, "f32"), (333, "u8"), (1024, "u8"), (40, "f32")):
        print(f"[noalloc] batch={batch} fmt={fmt}", flush=True)
        flat = torch.from_numpy(rng.integers(-3, rows + 3, batch).astype(np.int64)).to(dev)   # some rows out of range
        obs = torch.from_numpy(rng.integers(0, 4, batch).astype(np.int8)).to(dev)
        got = _outputs(dev, batch, fmt)
        torch.cuda.synchronize()
        free0, _ = torch.cuda.mem_get_info()
        _call(jq, L.lib.jq_history_reconstruct_noalloc, hist, flat, obs, fmt, got)
        torch.cuda.synchronize()
        free1, _ = torch.cuda.mem_get_info()
        want = _outputs(dev, batch, fmt)
        _call(jq, L.lib.jq_history_reconstruct, hist, flat, obs, fmt, want)
        torch.cuda.synchronize()
        for k in got:
            if got[k] is not None:
                assert torch.equal(got[k], want[k]), f"batch {batch} {fmt}: {k} differs"
        # every call, the first included: the library's code object is resident
        # (the rollout above launched its kernels), so any change is the call's own
        assert free0 == free1, f"batch {batch} {fmt}: device memory moved by {free0 - free1} bytes in the no-allocation call"
    big = torch.zeros(L.NOALLOC_MAX_ROWS + 1, dtype=torch.int64, device=dev)
    bobs = torch.zeros(L.NOALLOC_MAX_ROWS + 1, dtype=torch.int8, device=dev)
    out = _outputs(dev, 1, "f32")
    rc = L.lib.jq_history_reconstruct_noalloc(hist._h, big.data_ptr(), bobs.data_ptr(), big.numel(), L.OBS_F32,
                                              out["spatial"].data_ptr(), None, out["global"].data_ptr(), None, None,
                                              torch.cuda.current_stream().cuda_stream)
    assert rc == L.JQ_E_ARG and b"exceeds" in L.lib.jq_last_error()
    hist.close()
