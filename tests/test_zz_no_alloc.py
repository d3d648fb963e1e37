"""shv_hip_delta_rule_noalloc (the delta rule without any allocation: the chunked scan works in a static device
array of 16 windows) against shv_hip_delta_rule (which allocates its work buffer per call), through the C ABI.
Both run the same kernels in the same order, so outputs must be bitwise equal: in every tier and variant, for two
calls in a row -- the second with fewer windows, so a stale area from the first call cannot pass unnoticed -- and
past the limit the call is refused before any device work."""
import numpy as np
import pytest

from test_delta import H, T, inputs

pytestmark = pytest.mark.gpu

CASES = [("fp16", 0), ("fp16", 2), ("bf16", 0), ("bf16", 2), ("fp16", 1), ("fp32", 0), ("fp32", 1)]


@pytest.mark.parametrize("mode,variant", CASES)
def test_noalloc_matches_allocating_entry(shv, mode, variant):
    hip = shv.Hip()
    big, small = 16, 5
    q, k, v, dec, beta = inputs(big, 23)
    bufs = [hip.upload(x) for x in (q, k, v, dec, beta)]
    out_bytes = big * T * H * 128 * 4
    d_ref, d_got = hip.malloc(out_bytes), hip.malloc(out_bytes)
    stream = hip.stream()
    try:
        for n in (big, small):
            print(f"[gpu] delta rule no-alloc {mode} variant {variant}, {n} windows", flush=True)
            hip.memset(d_ref, 0xFF, out_bytes)
            hip.memset(d_got, 0xFF, out_bytes)
            shv.delta_rule(mode, *bufs, n, d_ref, variant)
            hip.sync()
            # inputs of the second call are the first call's leading windows: its area holds other windows' data
            shv.delta_rule_noalloc(mode, *bufs, n, d_got, variant, stream)
            hip.stream_sync(stream)
            ref = hip.download(d_ref, (n * T, H * 128), np.float32)
            got = hip.download(d_got, (n * T, H * 128), np.float32)
            assert np.all(np.isfinite(ref))
            assert np.array_equal(got.view(np.uint32), ref.view(np.uint32)), float(np.abs(got - ref).max())
    finally:
        hip.stream_destroy(stream)
        for p in bufs + [d_ref, d_got]:
            hip.free(p)


def test_noalloc_rejects_more_windows_than_its_area(shv):
    lib = shv.library()
    fake = 256   # never dereferenced: the size check comes first
    rc = lib.shv_hip_delta_rule_noalloc(b"fp16", fake, fake, fake, fake, fake, 17, fake, 0, None)
    assert rc == -1
    assert "exceed the static work area" in shv.last_error()
