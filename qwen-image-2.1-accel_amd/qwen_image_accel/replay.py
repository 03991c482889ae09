"""Teacher-forced replay: a profile's velocity error along the baseline's own
denoising path.

Reference interface: benchmarks/teacher_forced.py.  ``trace`` (:27-57) wraps
the pipeline's ``transformer.forward`` to record every velocity prediction and
its ``scheduler.step`` to record the latent each step produces -- or, when
replaying, to hand back a recorded latent in its place, so the candidate sees
exactly the inputs the baseline saw.  ``main`` (:60-110) traces the baseline
once per case, replays its latents through each candidate profile, and reports
the per-step relative RMSE of the velocity, ||v - v_ref||_2 / ||v_ref||_2
(:93-102: mean, max, first, last, per step).

Here the pipeline is any object with ``transformer.forward``,
``scheduler.step`` (returning a tuple whose first item is the latent, or an
object with ``prev_sample``) and a denoising loop started by ``run(pipe)``, so
the same code drives Diffusers' QwenImage21Pipeline on a box with the weights
and a stand-in pipeline elsewhere.
"""
import contextlib

import torch


class Recording:
    """What one traced run saw: the velocity of every transformer call (fp32,
    host), the latent every scheduler step produced (host, as produced; empty
    when replaying) and the number of scheduler steps taken."""

    def __init__(self):
        self.velocities = []
        self.latents = []
        self.steps = 0


def _sample_of(out):
    return out[0] if isinstance(out, tuple) else out.prev_sample


def _with_sample(out, sample):
    if isinstance(out, tuple):
        return (sample,) + tuple(out[1:])
    out.prev_sample = sample
    return out


@contextlib.contextmanager
def recording(pipe, replay=None):
    """Trace the pipeline inside the block (benchmarks/teacher_forced.py:27-57).
    With ``replay`` (a list of latents), step i returns ``replay[i]`` (moved to
    the produced latent's device and dtype) instead of what the scheduler
    produced; the produced latents are then not recorded.  The pipeline's
    methods are restored on exit, also after an error."""
    rec = Recording()
    transformer, scheduler = pipe.transformer, pipe.scheduler
    forward, step = transformer.forward, scheduler.step
    had_forward, had_step = "forward" in vars(transformer), "step" in vars(scheduler)

    def traced_forward(*args, **kwargs):
        out = forward(*args, **kwargs)
        rec.velocities.append(out[0].detach().float().cpu())
        return out

    def traced_step(*args, **kwargs):
        out = step(*args, **kwargs)
        produced = _sample_of(out)
        i = rec.steps
        rec.steps += 1
        if replay is None:
            rec.latents.append(produced.detach().cpu())
            return out
        if i >= len(replay):
            raise IndexError(f"replay holds {len(replay)} latents; the pipeline took step {i + 1}")
        return _with_sample(out, replay[i].to(produced.device, produced.dtype))

    transformer.forward, scheduler.step = traced_forward, traced_step
    try:
        yield rec
    finally:
        # drop the instance attributes again where the methods came from the class
        if had_forward:
            transformer.forward = forward
        else:
            del transformer.forward
        if had_step:
            scheduler.step = step
        else:
            del scheduler.step


def trace(pipe, run, replay=None):
    """One traced run: ``run(pipe)`` inside ``recording``.  Returns
    (velocities, latents) as benchmarks/teacher_forced.py:27 does."""
    with recording(pipe, replay) as rec:
        run(pipe)
        if torch.cuda.is_available():
            torch.cuda.synchronize()
    return rec.velocities, rec.latents


def relative_rmse(reference, candidate):
    """Per-step ||c - r||_2 / ||r||_2 of two velocity lists and its summary
    (benchmarks/teacher_forced.py:93-102).  The RMS ratio is computed in
    float64 so that a zero difference reads exactly 0."""
    if len(reference) != len(candidate) or not reference:
        raise ValueError(f"velocity lists differ in length or are empty ({len(reference)} vs {len(candidate)})")
    errors = []
    for r, c in zip(reference, candidate):
        r64, c64 = r.double(), c.double()
        errors.append(float((c64 - r64).pow(2).mean().sqrt() / r64.pow(2).mean().sqrt()))
    return {"relative_rmse_mean": sum(errors) / len(errors), "relative_rmse_max": max(errors),
            "relative_rmse_first": errors[0], "relative_rmse_last": errors[-1],
            "per_step": [round(e, 6) for e in errors]}


def teacher_forced(make_pipe, profiles, cases, baseline="baseline"):
    """The replay experiment of benchmarks/teacher_forced.py:60-110 without its
    command line: ``make_pipe(profile)`` builds a configured pipeline,
    ``cases`` maps a case name to ``run(pipe)``.  The baseline is traced once
    per case; each profile replays the baseline's latents.  Returns
    {profile: {case: relative_rmse(...)}}."""
    pipe = make_pipe(baseline)
    reference = {name: trace(pipe, run) for name, run in cases.items()}
    del pipe
    report = {}
    for profile in profiles:
        pipe = make_pipe(profile)
        report[profile] = {name: relative_rmse(reference[name][0], trace(pipe, run, replay=reference[name][1])[0])
                           for name, run in cases.items()}
        del pipe
    return report
