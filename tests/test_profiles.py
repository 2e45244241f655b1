"""The committed profiles carry what bench.py reads from them: the per-launch HBM traffic totals of the attention
kernel and of the selection (rocprofv3 FETCH_SIZE / WRITE_SIZE), and every summary names the command that made it
(rocprofv3, or a committed entry point: bench.py, python -m streamvoxel_amd....)."""
import os
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)


def test_traffic_totals_are_present_and_plausible():
    import bench
    attn = bench.profiled_traffic('xattn_fwd_kernel')
    select = bench.profiled_traffic('ease_select')
    assert attn is not None and select is not None
    # Algorithmic bytes of the bench workload: attention 173.4 MB (Q, K/V once, O), selection 542.1 MB; the HBM
    # traffic cannot be below them and should not be far above.
    assert 173.4e6 <= attn <= 1.2 * 173.4e6
    assert 542.1e6 <= select <= 1.2 * 542.1e6


def test_every_profile_names_its_command():
    d = os.path.join(ROOT, 'profiles')
    names = sorted(f for f in os.listdir(d) if f.endswith(('.md', '.txt')))
    assert names
    for name in names:
        with open(os.path.join(d, name)) as f:
            text = f.read()
        # a rocprofv3 summary, or a timing summary made by a committed entry point of this repository
        assert any(cmd in text for cmd in ('rocprofv3', 'python -m streamvoxel_amd.', 'bench.py')), name
        assert '```' in text, name
