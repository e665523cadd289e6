"""The selector's initial weights equal the reference's, bit for bit.

Fixtures: ``tests/golden/selector_init.{json,safetensors}``, written by
``tests/golden/make_selector_init.py`` from the reference's own
``LeanSelectSelector.reset_parameters`` (leanselect/selector.py:112-137) under
fixed seeds, for router widths below, equal to and above head_dim.
"""
import json
from pathlib import Path

import pytest
import torch
from safetensors.torch import load_file

from leanselect_amd.selector import LeanSelectSelector

GOLDEN = Path(__file__).resolve().parent / "golden"
META = json.loads((GOLDEN / "selector_init.json").read_text())
TENSORS = load_file(str(GOLDEN / "selector_init.safetensors"))


@pytest.mark.parametrize("case", META["cases"], ids=[c["name"] for c in META["cases"]])
def test_reset_parameters_matches_reference(case):
    torch.manual_seed(case["seed"])
    sel = LeanSelectSelector(num_heads=case["num_heads"], num_kv_heads=case["num_kv_heads"],
                             head_dim=case["head_dim"], router_heads=case["router_heads"],
                             router_dim=case["router_dim"])
    for name in ("head_mix", "kv_head_mix", "q_proj", "k_proj"):
        want = TENSORS[f"{case['name']}.{name}"]
        got = getattr(sel, name).detach()
        assert got.shape == want.shape and got.dtype == want.dtype, name
        assert torch.equal(got, want), f"{case['name']}.{name}"


def test_fixture_catches_a_changed_draw():
    """The comparison is sensitive to the draw: another seed's frame differs."""
    case = META["cases"][0]
    torch.manual_seed(case["seed"] + 100)
    sel = LeanSelectSelector(num_heads=case["num_heads"], num_kv_heads=case["num_kv_heads"],
                             head_dim=case["head_dim"], router_heads=case["router_heads"],
                             router_dim=case["router_dim"])
    assert not torch.equal(sel.q_proj.detach(), TENSORS[f"{case['name']}.q_proj"])
