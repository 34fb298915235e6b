"""Tolerance checks shared by the GPU parity tests.

Float atomics make the raster gradients order-dependent, so they cannot be
bit-exact.  The checks here bound every element by the rounding error that
summation order and per-summand rounding can cause, and carry that bound
through the rest of the step:

  raster gradients   |g - o| <= 1e-3 |o| + 1e-4 A + 1e-7 max|o|, with A (from
                     the oracle) the sum of the magnitudes of the parts the
                     element's summands are formed from, and max|o| over
                     the component;
  parameter grads    the projection backward is linear in the raster
                     gradients, so their allowed error is that bound pushed
                     through it (estimated with random-sign probes);
  post-Adam params   Adam's first step moves an element by lr * g / (|g| +
                     eps): every parameter within the range of steps its
                     gradient's allowed error permits, which is below 1e-5
                     wherever that gradient is resolved (its sign and size
                     determined beyond the noise); elsewhere the step is
                     rounding noise, up to 2 lr.
"""
from __future__ import annotations

import json
import os

import numpy as np

RTOL, CTOL, FLOOR = 1e-3, 1e-4, 1e-7


def record(kind: str, what: str, **vals) -> None:
    """Appends one JSON line {kind, what, ...} to the file named by
    MSPLAT_PARITY_LOG, if set: how far the literal bars (gradients within
    1e-3 relative, post-Adam parameters within 1e-5) hold on a run."""
    path = os.environ.get("MSPLAT_PARITY_LOG")
    if not path:
        return
    with open(path, "a") as f:
        f.write(json.dumps(dict(kind=kind, what=what, **vals)) + "\n")


def literal_rel(g, o, rtol=1e-3):
    """The elements of g outside rtol |o| of o: count, and the same among
    the significant elements (|o| above 1e-3 of the component's or array's
    largest magnitude), with the worst relative error there."""
    g = np.asarray(g, np.float64)
    o = np.asarray(o, np.float64)
    err = np.abs(g - o)
    miss = err > rtol * np.abs(o)
    scale = np.abs(o).max(axis=0) if o.ndim == 2 else np.abs(o).max()
    sig = np.abs(o) > 1e-3 * scale
    rel = np.where(sig, err / np.maximum(np.abs(o), 1e-300), 0.0)
    return dict(elements=int(o.size), beyond_1e3_rel=int(miss.sum()), significant=int(sig.sum()),
                significant_beyond_1e3_rel=int((miss & sig).sum()), worst_rel_significant=float(rel.max()))


def raster_bound(o, a):
    """Allowed error of each raster-gradient element [N,16]: rtol |o| +
    ctol A, plus a floor of 1e-7 of the component's largest magnitude (a
    gradient 10^7 times smaller than its component's scale has no relative
    accuracy to check: its summands are formed from rays and transmittances
    whose own rounding is not small against it)."""
    o = np.abs(np.asarray(o, np.float64))
    return RTOL * o + CTOL * np.asarray(a, np.float64) + FLOOR * o.max(axis=0) + 1e-30


def grad_close(g, o, a, what):
    """Per element |g - o| <= raster_bound(o, A).  An element whose summands
    do not cancel (A = |o|) is held to about 1.1e-3 relative.  Prints how
    many elements pass only through the floor, and how many miss the
    tighter |g - o| <= 1e-4 |o| + 1e-6 max|o|."""
    g = np.asarray(g, np.float64)
    o = np.asarray(o, np.float64)
    a = np.asarray(a, np.float64)
    err = np.abs(g - o)
    bound = raster_bound(o, a)
    ratio = err / bound
    bad = ratio > 1.0
    floor_only = err > RTOL * np.abs(o) + CTOL * a
    tight = err > 1e-4 * np.abs(o) + 1e-6 * np.abs(o).max(axis=0)
    record("raster_grads", what, worst_err_over_bound=float(ratio.max()), **literal_rel(g, o))
    print(f"[grad] {what}: worst err/bound {ratio.max():.3g}, misses {int(bad.sum())} of {bad.size}, "
          f"within the floor only {int((floor_only & ~bad).sum())}; outside 1e-4|o| + 1e-6 max|o|: "
          f"{int(tight.sum())} per component {tight.sum(axis=0).tolist()}", flush=True)
    if bad.any():
        i = np.unravel_index(np.argmax(ratio), ratio.shape)
        raise AssertionError(f"{what}: {int(bad.sum())} elements outside their bound; worst at {i}: gpu {g[i]!r} "
                             f"oracle {o[i]!r} A {a[i]!r}")


def param_grad_noise(orc, params: dict, cam, degree, dtu, radii, g16_o, a16_o, probes=4, seed=0):
    """Allowed error of each parameter gradient: the raster-gradient bound
    pushed through the oracle's projection backward (linear
    in its raster-gradient input) with random signs, the largest of
    `probes` probes times 4 (the opacity gradient is the raster component
    itself, so its bound is exact).  Returns the six groups (means, scales, quats,
    features_dc, features_rest, opacities) as flat arrays."""
    b16 = raster_bound(g16_o, a16_o).astype(np.float32)
    rng = np.random.default_rng(seed)
    n = b16.shape[0]
    worst = None
    for _ in range(probes):
        probe = (b16 * rng.choice(np.float32([-1.0, 1.0]), size=b16.shape)).astype(np.float32)
        out = orc.project_bwd(params, cam, degree, dtu, radii, probe,
                              dict(grad_norm=np.zeros(n, np.float32), vis=np.zeros(n, np.float32),
                                   max2d=np.zeros(n, np.float32)))
        groups = [out["dmeans"], out["dscales"], out["dquats"], out["dfdc"], out["dfrest"]]
        groups = [np.abs(x.astype(np.float64)).reshape(-1) for x in groups]
        worst = groups if worst is None else [np.maximum(w, x) for w, x in zip(worst, groups)]
    # the opacity gradient is the raster component itself: its bound exactly
    return [4.0 * w for w in worst] + [b16[:, 12].astype(np.float64)]


def adam_first_step(g, lr, eps=1e-8):
    """The step Adam's first update takes for gradient g: with m = (1 -
    beta1) g, v = (1 - beta2) g^2 and both bias corrections, it is
    lr * g / (|g| + eps)."""
    return lr * g / (np.abs(g) + eps)


def post_adam_close(names, got_params, orc_params, got_m, orc_m, noise, lrs, beta1=0.9, label=""):
    """First Adam step.  Parameter gradients (recovered from the first
    moments, m = (1 - beta1) g) must lie within their allowed error; every
    parameter must lie within the range of steps that error allows, i.e.
    |p - p_o| <= max over g in [g_o - e, g_o + e] of |step(g) - step(g_o)|.
    That range is below 1e-5 wherever the gradient is resolved; the elements
    where it is not (|g_o| near the noise or near eps) are counted."""
    for name, p, po, m, mo, nz, lr in zip(names, got_params, orc_params, got_m, orc_m, noise, lrs):
        p = np.asarray(p, np.float64).reshape(-1)
        po = np.asarray(po, np.float64).reshape(-1)
        g = np.asarray(m, np.float64).reshape(-1) / (1.0 - beta1)
        go = np.asarray(mo, np.float64).reshape(-1) / (1.0 - beta1)
        # one ulp of the moment itself on top of the propagated bound
        allowed = nz + RTOL * np.abs(go) + 2.5e-7 * np.abs(go) + 1e-30
        gerr = np.abs(g - go)
        assert (gerr <= allowed).all(), (
            f"{name}: {int((gerr > allowed).sum())} parameter gradients outside their allowed error; worst ratio "
            f"{(gerr / allowed).max():.3g}")
        s0 = adam_first_step(go, lr)
        reach = np.maximum(np.abs(adam_first_step(go + allowed, lr) - s0),
                           np.abs(adam_first_step(go - allowed, lr) - s0))
        # plus the float rounding of the parameter update itself
        limit = reach + 2.5e-7 * np.maximum(np.abs(po), 1.0)
        diff = np.abs(p - po)
        unresolved = reach > 1e-5
        record("param_grads", f"{label} {name}".strip(), **literal_rel(g, go))
        record("post_adam", f"{label} {name}".strip(), elements=int(p.size), beyond_1e5=int((diff > 1e-5).sum()),
               max_abs_diff=float(diff.max()), unresolved=int(unresolved.sum()),
               beyond_1e5_resolved=int(((diff > 1e-5) & ~unresolved).sum()))
        print(f"[adam] {name}: {int(unresolved.sum())} of {p.size} steps not resolved to 1e-5 by the gradient's "
              f"allowed error; {int((diff > 1e-5).sum())} parameters beyond 1e-5 (max {diff.max():.3g}); "
              f"worst diff/limit {(diff / limit).max():.3g}", flush=True)
        bad = diff > limit
        assert not bad.any(), (f"{name}: {int(bad.sum())} parameters outside the range their gradient's allowed "
                               f"error permits, worst ratio {(diff / limit).max():.3g}")
        assert not (diff > 1e-5)[~unresolved].any()


def trainer_post_adam_close(name, got, orc, orc_m, lr, beta1=0.9, eps=1e-8):
    """One trainer step against the golden model's step, per element, from
    the golden model's first moments alone (the trainer keeps its gradients
    on the GPU): with g_o = m_o / (1 - beta1), a gradient error of up to
    RTOL |g_o| + FLOOR max|g_o| (float-atomic order, the GPU backward's
    hardware exp2 against the golden model's Gaussian) moves Adam's first
    step by at most reach = max |step(g_o +- err) - step(g_o)|.  Every
    parameter must lie within max(1e-5 max(1, max|p|), reach + its own
    rounding): the plain 1e-5 bar wherever the gradient is resolved."""
    p = np.asarray(got, np.float64).reshape(-1)
    po = np.asarray(orc, np.float64).reshape(-1)
    go = np.asarray(orc_m, np.float64).reshape(-1) / (1.0 - beta1)
    err = RTOL * np.abs(go) + FLOOR * np.abs(go).max() + 1e-30
    s0 = adam_first_step(go, lr, eps)
    reach = np.maximum(np.abs(adam_first_step(go + err, lr, eps) - s0), np.abs(adam_first_step(go - err, lr, eps) - s0))
    bar = 1e-5 * max(1.0, np.abs(po).max())
    limit = np.maximum(bar, reach + 2.5e-7 * np.maximum(np.abs(po), 1.0))
    diff = np.abs(p - po)
    print(f"[adam] {name}: max diff {diff.max():.3g}, {int((diff > bar).sum())} of {p.size} beyond 1e-5 "
          f"(all within their gradient's reach: {bool((diff <= limit).all())})", flush=True)
    assert (diff <= limit).all(), (
        f"{name}: {int((diff > limit).sum())} parameters outside their reach; worst ratio {(diff / limit).max():.3g}")
