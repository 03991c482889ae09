"""Teacher-forced replay (benchmarks/teacher_forced.py) on the CPU with the
stand-in pipeline: the error metric against closed forms, the forcing of the
latents, and the restoring of the pipeline's methods."""
import pytest
import torch

from qwen_image_accel import pipeline, replay
from tests import fake_qwen21 as fq


def _run(latents):
    return lambda pipe: pipe(latents.clone())


def test_relative_rmse_closed_form():
    """c = r (1 + e_i) gives exactly |e_i| per step."""
    g = torch.Generator().manual_seed(3)
    ref = [torch.randn(4, 33, generator=g, dtype=torch.float64) for _ in range(4)]
    eps = [0.0, 1e-3, -0.25, 0.5]
    rep = replay.relative_rmse(ref, [r * (1 + e) for r, e in zip(ref, eps)])
    assert rep["relative_rmse_first"] == 0.0
    assert rep["relative_rmse_max"] == pytest.approx(0.5, rel=1e-12)
    assert rep["relative_rmse_last"] == pytest.approx(0.5, rel=1e-12)
    assert rep["relative_rmse_mean"] == pytest.approx(sum(abs(e) for e in eps) / 4, rel=1e-12)
    assert rep["per_step"] == [0.0, 0.001, 0.25, 0.5]
    # an orthogonal error of the same norm: sqrt(2) - 1 would be wrong, 1 is right
    r = torch.tensor([[1.0, 0.0]])
    assert replay.relative_rmse([r], [torch.tensor([[1.0, 1.0]])])["relative_rmse_max"] == 1.0
    with pytest.raises(ValueError):
        replay.relative_rmse(ref, ref[:2])


def test_trace_records_every_step_and_restores():
    pipe, x0 = fq.make_pipeline(steps=5)
    with torch.no_grad():
        vel, lat = replay.trace(pipe, _run(x0))
    assert len(vel) == 5 and len(lat) == 5
    assert "forward" not in vars(pipe.transformer) and "step" not in vars(pipe.scheduler)
    # the recorded latents are the sampler's own: x_{i+1} = x_i + dt_i v_i
    x = x0
    for i in range(5):
        dt = float(pipe.scheduler.sigmas[i + 1] - pipe.scheduler.sigmas[i])
        x = (x.float() + dt * vel[i]).to(x0.dtype)
        assert torch.equal(x, lat[i])


def test_replay_forces_the_baseline_latents():
    """A candidate whose own sampler drifts still sees the baseline's latents:
    its velocities equal the baseline's bit for bit (error exactly 0)."""
    base, x0 = fq.make_pipeline(steps=4)
    cand, _ = fq.make_pipeline(steps=4)
    step = cand.scheduler.step
    cand.scheduler.step = lambda v, i, s: ((step(v, i, s)[0].float() * 1.5).to(s.dtype),)
    with torch.no_grad():
        vel, lat = replay.trace(base, _run(x0))
        free, _ = replay.trace(cand, _run(x0))
        forced, none = replay.trace(cand, _run(x0), replay=lat)
    assert none == []
    assert replay.relative_rmse(vel, free)["relative_rmse_max"] > 0.01
    assert replay.relative_rmse(vel, forced)["relative_rmse_max"] == 0.0
    assert "step" in vars(cand.scheduler)   # an instance attribute before tracing stays one


def test_replay_too_short_raises_and_restores():
    pipe, x0 = fq.make_pipeline(steps=3)
    with torch.no_grad():
        _, lat = replay.trace(pipe, _run(x0))
        with pytest.raises(IndexError, match="replay holds 2"):
            replay.trace(pipe, _run(x0), replay=lat[:2])
    assert "forward" not in vars(pipe.transformer) and "step" not in vars(pipe.scheduler)


def test_teacher_forced_fused_on_cpu_is_exact():
    """On CPU tensors the fused profile's kernels take the eager fallbacks, so
    its replay error is exactly 0 (the reference reports 0 for `fused`)."""
    def make(profile):
        pipe, _ = fq.make_pipeline(steps=3)
        pipeline.install_hot_path(pipe.transformer, profile, validate=False)
        return pipe

    _, x0 = fq.make_pipeline(steps=3)
    with torch.no_grad():
        rep = replay.teacher_forced(make, ["fused"], {"a": _run(x0), "b": _run(-x0)})
    assert set(rep) == {"fused"} and set(rep["fused"]) == {"a", "b"}
    for case in rep["fused"].values():
        assert case["relative_rmse_max"] == 0.0 and len(case["per_step"]) == 3



class _Out:
    def __init__(self, sample):
        self.prev_sample = sample


class _ObjScheduler(fq.FlowEulerScheduler):
    """Returns an object with `prev_sample`, as Diffusers' schedulers do unless
    return_dict=False; `factor` makes a drifting sampler."""

    def __init__(self, steps, factor=1.0):
        super().__init__(steps)
        self.factor = factor

    def step(self, velocity, index, sample):
        x = super().step(velocity, index, sample)[0]
        return _Out((x.float() * self.factor).to(sample.dtype))


class _ObjPipeline(fq.StandInPipeline):
    def __call__(self, latents):
        for i in range(self.steps):
            v = self.transformer(latents, float(self.scheduler.sigmas[i]))[0]
            latents = self.scheduler.step(v, i, latents).prev_sample
        return latents


def test_scheduler_output_objects_are_forced_too():
    """Replay replaces `prev_sample` on a scheduler output object."""
    pipes = []
    for factor in (1.0, 0.5):
        p, x0 = fq.make_pipeline(steps=3)
        obj = _ObjPipeline(p.transformer, 3)
        obj.scheduler = _ObjScheduler(3, factor)
        pipes.append(obj)
    base, cand = pipes
    with torch.no_grad():
        vel, lat = replay.trace(base, _run(x0))
        free, _ = replay.trace(cand, _run(x0))
        forced, _ = replay.trace(cand, _run(x0), replay=lat)
    assert len(lat) == 3 and all(isinstance(t, torch.Tensor) for t in lat)
    assert replay.relative_rmse(vel, free)["relative_rmse_max"] > 0.01
    assert replay.relative_rmse(vel, forced)["relative_rmse_max"] == 0.0


def test_configure_pipeline_needs_a_gpu_for_kernel_profiles():
    """configure_pipeline (pipeline.py:109-198) validates before it changes
    anything: without a ROCm GPU the kernel profiles are refused and the
    pipeline stays unconfigured."""
    if torch.cuda.is_available():
        pytest.skip("checks the CPU-only refusal")
    pipe, _ = fq.make_pipeline(steps=2)
    for profile in ("fused", "mxfp8"):
        with pytest.raises(RuntimeError, match="ROCm GPU"):
            pipeline.configure_pipeline(pipe, profile)
    assert not hasattr(pipe, "_qw_optimization") and "_qw_hot_path" not in vars(pipe.transformer)
