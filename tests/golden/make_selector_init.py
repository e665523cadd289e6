"""Write the initial selector weights of the reference's ``LeanSelectSelector``.

``reset_parameters`` (leanselect/selector.py:112-137) draws a QR frame from
torch's RNG, so no closed form pins its values.  This script loads the
reference's selector module by file path (it imports only torch), builds the
selector under fixed seeds for three geometries (router width below, equal to
and above head_dim, which takes the transposed-QR branch) and stores the four
master tensors in ``selector_init.safetensors``, with the seed and geometry of
each case in ``selector_init.json``.  It runs only where the LeanSelect
repository is checked out; the tests read the fixtures.

Usage: python tests/golden/make_selector_init.py [/path/to/LeanSelect]
"""
import sys

# Executing the reference module must leave no bytecode beside its source.
sys.dont_write_bytecode = True

import importlib.util  # noqa: E402
import json  # noqa: E402
from pathlib import Path  # noqa: E402

import torch  # noqa: E402
from safetensors.torch import save_file  # noqa: E402

CASES = [
    # name, num_heads, num_kv_heads, head_dim, router_heads, router_dim, seed
    ("h8_g2_d128_r4x32", 8, 2, 128, 4, 32, 0),
    ("h16_g4_d64_r2x16", 16, 4, 64, 2, 16, 1),
    ("h32_g2_d64_r4x32", 32, 2, 64, 4, 32, 2),
]


def main() -> None:
    root = Path(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
    spec = importlib.util.spec_from_file_location("ref_selector", root / "leanselect" / "selector.py")
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    tensors, meta = {}, []
    for name, H, G, D, R, F, seed in CASES:
        torch.manual_seed(seed)
        sel = mod.LeanSelectSelector(num_heads=H, num_kv_heads=G, head_dim=D, router_heads=R,
                                     router_dim=F)
        for t in ("head_mix", "kv_head_mix", "q_proj", "k_proj"):
            tensors[f"{name}.{t}"] = getattr(sel, t).detach().clone().contiguous()
        meta.append(dict(name=name, num_heads=H, num_kv_heads=G, head_dim=D, router_heads=R,
                         router_dim=F, seed=seed))
    here = Path(__file__).resolve().parent
    save_file(tensors, str(here / "selector_init.safetensors"))
    (here / "selector_init.json").write_text(json.dumps(
        {"source": "leanselect/selector.py:112-137 (LeanSelectSelector.reset_parameters)",
         "torch": torch.__version__, "cases": meta}, indent=1))
    print(here / "selector_init.safetensors")


if __name__ == "__main__":
    main()
