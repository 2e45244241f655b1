"""Reveal schedules (host integers), same API as streamvoxel/sampling/schedule.py:1-38."""
import math


def actual_time(mask_fraction):
    """Masked fraction -> model time (streamvoxel/sampling/schedule.py:4-5)."""
    return 2 * math.asin(min(1., max(0., mask_fraction))) / math.pi


def reveal_fraction(u, schedule):
    """streamvoxel/sampling/schedule.py:8-12."""
    if schedule == 'linear':
        return u
    if schedule == 'halfcos':
        return (1 - math.cos(math.pi * u)) / 2
    if schedule == 'reversequarter':
        return math.sin(math.pi * u / 2)
    raise ValueError(schedule)


def quota_counts(total, steps, schedule):
    """Legacy rounding: cumulative floor(total * f(s/steps) + 1e-9) (streamvoxel/sampling/schedule.py:15-18)."""
    cumulative = [0]
    for s in range(1, steps + 1):
        cumulative.append(min(total, max(0, math.floor(total * reveal_fraction(s / steps, schedule) + 1e-9))))
    cumulative[-1] = total
    return [hi - lo for lo, hi in zip(cumulative, cumulative[1:])]


_CURVES = {
    'linear': lambda u: u,
    'quartercos': lambda u: 1 - math.cos(math.pi * u / 2),
    'reversequarter': lambda u: math.sin(math.pi * u / 2),
    'halfcos': lambda u: (1 - math.cos(math.pi * u)) / 2,
    'arccos': lambda u: 2 / math.pi * math.acos(1 - u),
}


def curve(u, name):
    """Cumulative reveal curve on [0, 1] (streamvoxel/sampling/schedule.py:21-29); 'front<p>' / 'power<p>' are
    the power families 1-(1-u)^p and u^p."""
    if name in _CURVES:
        return _CURVES[name](u)
    if name.startswith('front'):
        return 1 - (1 - u) ** float(name[5:])
    if name.startswith('power'):
        return u ** float(name[5:])
    raise ValueError(name)


def counts(total, spec):
    """Per-step reveal counts (streamvoxel/sampling/schedule.py:32-38). 'positive' rounding (the default) adds one
    voxel per step under the curve, so every step reveals at least one; 'legacy' uses `quota_counts`."""
    if spec['schedule'] == 'native_quarter':
        return None
    if spec.get('rounding') == 'legacy':
        return quota_counts(total, spec['steps'], spec['schedule'])
    steps = spec['steps']
    if not 1 <= steps <= total:
        raise AssertionError((total, steps))
    spread = total - steps
    cumulative = [0] + [s + math.floor(spread * curve(s / steps, spec['schedule']) + 1e-10) for s in range(1, steps + 1)]
    cumulative[-1] = total
    q = [hi - lo for lo, hi in zip(cumulative, cumulative[1:])]
    if min(q) < 1 or sum(q) != total:
        raise AssertionError(q)
    return q
