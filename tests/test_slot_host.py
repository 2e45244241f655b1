"""Host-side logic of the product slot module against the oracle (no GPU): ForwardBudget's forward counting."""
from oracle.slot import ForwardBudget as OracleBudget
from streamvoxel_amd.stream.slot import ForwardBudget


def test_forward_budget_matches_oracle():
    for total in (1, 2, 5, 26):
        a, b = ForwardBudget(), OracleBudget()
        assert a.forward() == b.forward() is False
        a.arm(total)
        b.arm(total)
        for _ in range(total + 3):
            assert a.forward() == b.forward()
            assert (a.phase, a.left, a.nfe) == (b.phase, b.left, b.nfe)
        assert a.phase == 'idle'


def test_forward_budget_rejects_empty_window():
    import pytest
    with pytest.raises(ValueError):
        ForwardBudget().arm(0)
