"""The op-by-op device route as a network: the sequence of C-ABI calls that
integration/csharp/HipBackend.cs issues when the reference's PtModel.Run walks
a YOLOv8 model on the HIP device (per conv: op-23 NCHW -> NHWC, sy_conv_run,
op-23 back; op-10 shortcuts, op-21 pools, op-20 upsamples, op-26 concats,
op-24 slices or borrowed views, op-30 per level into the joined head), with
the graph replay that backend rebuilds on sy_graph_* (VulkanReplay.cs:31-129):
frame 1 eager, frame 2 captured and launched, frame 3 replayed.

Bars as for the fused model path: raw head within max-rel 1e-3 of the
oracle on every image, NMS index sets equal except near-ties; the eager,
captured and replayed frames of one input are bit-identical.
"""
import numpy as np
import pytest

import oracle
from simdyolo_amd import synth
from simdyolo_amd.device_route import DeviceRouteDetector, HipDeviceBackend, binary, parameters
from _parity import adaptive_threshold, check_detections, max_rel

pytestmark = pytest.mark.gpu

HEAD_TOL = 1e-3


@pytest.mark.timeout(600)
@pytest.mark.parametrize("batch", [1, 32])
def test_route_yolov8n_640_against_oracle(batch):
    cfg = synth.config("n")
    params = synth.params(cfg)
    x = synth.images(batch, 640, 640)
    print(f"device route YOLOv8n 640 batch {batch}", flush=True)
    with DeviceRouteDetector(cfg, params) as det:
        frames = [det.predict_raw(x) for _ in range(3)]
        replayed = det.backend.replayed_frames
    assert replayed == 1, "frame 3 was not a graph replay"
    for f in frames[1:]:
        assert f.tobytes() == frames[0].tobytes(), "eager, captured and replayed frames differ"
    got = frames[-1]
    assert got.shape == (batch, 84, 8400)
    exp = oracle.yolov8_forward(params, x)
    worst = max(max_rel(got[i], exp[i]) for i in range(batch))
    print(f"  worst max-rel {worst:.3e} over {batch} images", flush=True)
    assert worst <= HEAD_TOL
    n_got, n_exp = check_detections(got[0], exp[0], conf=adaptive_threshold(exp[0]))
    assert n_exp >= 10


@pytest.mark.timeout(300)
def test_route_replay_takes_new_input(tmp_path):
    """A replay reads the new frame's input: its head equals an eager frame of
    that input on a backend without replay.  The second backend loads the
    first one's tuning table, so both run the same kernel for every conv
    (the tuner picks by timing, and candidates differ in summation order)."""
    cfg = synth.config("n")
    params = synth.params(cfg)
    xs = [synth.images(2, 320, 320, seed=synth.SEED + j) for j in range(4)]
    table = str(tmp_path / "tune.txt")
    with DeviceRouteDetector(cfg, params) as det:
        got = [det.predict_raw(x) for x in xs]
        assert det.backend.replayed_frames == 2
        det.backend.ctx.tune_save(table)
    with DeviceRouteDetector(cfg, params, replay=False) as ref:
        ref.backend.ctx.tune_load(table)
        exp = [ref.predict_raw(x) for x in xs]
        assert ref.backend.replayed_frames == 0
    for g, e in zip(got, exp):
        assert g.tobytes() == e.tobytes()


def test_route_capture_ends_on_host_upload():
    """Frame 1 qualifies for replay (its only host upload is the input);
    frame 2 is captured but needs a second host upload, so its capture ends
    there (the work recorded so far runs once) and it finishes op by op;
    frame 3 runs eagerly.  Every frame equals the same frame on a backend
    without replay, and nothing is replayed."""
    rng = np.random.Generator(np.random.PCG64(7))
    x = rng.standard_normal((2, 8, 16, 16)).astype(np.float32)
    extra = rng.standard_normal((2, 8, 16, 16)).astype(np.float32)

    def frame(be, second):
        be.begin_frame()
        try:
            be.begin_replay_capture(x)
            a = be.compute(1, [x], x.shape, parameters(x.size, 0), x.size)        # SiLU
            b = be.upload(second) if second is not None else a                     # a second host tensor
            y = binary(be, a, b, 12)
            return be.materialize_outputs([y])[0]
        finally:
            be.end_frame()

    plan = [None, extra, None]
    with HipDeviceBackend(0) as be:
        got = [frame(be, e) for e in plan]
        assert be.replayed_frames == 0
    with HipDeviceBackend(0, replay=False) as be:
        exp = [frame(be, e) for e in plan]
    for g, e in zip(got, exp):
        assert g.tobytes() == e.tobytes()
