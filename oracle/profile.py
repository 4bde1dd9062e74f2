"""CPU restatement of the structural layer-budget profile.

TEST INFRASTRUCTURE (see ``oracle/__init__.py``).

Follows ``evaluate.py:16-32`` of the reference with the constants of
``configs/paper.json:5-11``: when ``s > 0.70`` the favoured layers get
``s - 0.05`` and the others ``s + 6*0.05/(L-6)``; values are serialised with
``%.10f`` and parsed back as floats (``evaluate.py:32, 42``). The per-layer
QK budget is ``int(Kb*(1-s))``, at least 1 (``SW:1226-1228``,
``spas_sage_attn/utils.py:289``).

Pinning: ``tests/test_oracle_misc.py`` replays the reference's
``tests/test_release.py:43-51, 109-121`` assertions (24/18 values, mean equal
to ``s`` to 1e-9, favoured layer ``s-0.05``, ``None`` at 0.65 and 0.70,
active at 0.7001, ValueError when the profile leaves [0,1)) and the per-layer
budgets of the benchmark configurations worked out by hand (C2: 155/120
blocks, C3: 362/224, C4: 310/233).
"""
from __future__ import annotations

PAPER = {
    "enable_above": 0.70,
    "delta": 0.05,
    "vggt": {"layers": 24, "favored": (11, 12, 13, 14, 15, 16)},
    "pi3": {"layers": 18, "favored": (12, 13, 14, 15, 16, 17)},
}


def layer_sparsity(backbone: str, sparsity: float, allocation: str = "paper"):
    if backbone not in ("vggt", "pi3") or allocation not in ("paper", "uniform"):
        raise ValueError("unsupported backbone or allocation")
    if not 0 <= sparsity < 1:
        raise ValueError("sparsity must be in [0, 1)")
    if allocation == "uniform" or sparsity <= PAPER["enable_above"]:
        return None
    shape = PAPER[backbone]
    fav = shape["favored"]
    delta = PAPER["delta"]
    offset = len(fav) * delta / (shape["layers"] - len(fav))
    values = [sparsity - delta if i in fav else sparsity + offset for i in range(shape["layers"])]
    if any(not 0 <= x < 1 for x in values):
        raise ValueError("structural profile leaves [0, 1)")
    return [float(f"{x:.10f}") for x in values]


def budget(key_blocks: int, sparsity: float) -> int:
    return max(int(key_blocks * (1 - sparsity)), 1)
