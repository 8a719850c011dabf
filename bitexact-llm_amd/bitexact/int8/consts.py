"""int8-engine constants (src/bitexact/int8/consts.py:26-53): fractional bits and the exp table."""

import torch

FR = 16          # residual stream, layer outputs, logits
FG = 12          # RMSNorm gamma
FA = 12          # LUT input step (exp, SiLU)
FE = 30          # exp table values
FT = 16          # cos / sin
EXP_MIN = -32    # exp table domain [EXP_MIN, 0]


def exp_table(device=None):
    """e^x at FE bits for x = EXP_MIN .. 0 at step 2^-FA (2^17 + 1 entries; offline constant, float64 rounded
    once, src/bitexact/int8/consts.py:50-53)."""
    xs = torch.arange(EXP_MIN << FA, 1, dtype=torch.float64) / (1 << FA)
    t = torch.round(torch.exp(xs) * (1 << FE)).long()
    return t if device is None else t.to(device)
