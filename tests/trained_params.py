"""Parameter values a trained checkpoint would hold, for parity tests.

A freshly initialised mixer has A_log = 0 and every norm weight 1, so a test
built at init never exercises the per-head gate scale exp(A_log) or the norm
weights.  ``perturb_like_trained`` draws them away from their init values
(seeded), in place: A_log ~ N(0, 0.5^2), dt_bias += N(0, 0.3^2), every
``*norm.weight`` ~ U[0.5, 1.5].
"""

from __future__ import annotations

import torch


def perturb_like_trained(module: torch.nn.Module, seed: int) -> list[str]:
    gen = torch.Generator().manual_seed(seed)
    touched = []
    with torch.no_grad():
        for name, p in module.named_parameters():
            if name.endswith("A_log"):
                new = torch.randn(p.shape, generator=gen) * 0.5
            elif name.endswith("dt_bias"):
                new = p.detach().cpu() + torch.randn(p.shape, generator=gen) * 0.3
            elif name.endswith("norm.weight"):
                new = torch.rand(p.shape, generator=gen) + 0.5
            else:
                continue
            p.copy_(new.to(device=p.device, dtype=p.dtype))
            touched.append(name)
    return touched
