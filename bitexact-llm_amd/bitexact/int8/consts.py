"""int8-engine constants (src/bitexact/int8/consts.py:26-53, 79-80): fractional bits, the exp and SiLU tables."""

import torch

FR = 16          # residual stream, layer outputs, logits
FG = 12          # RMSNorm gamma
FA = 12          # LUT input step (exp, SiLU)
FE = 30          # exp table values
FT = 16          # cos / sin
EXP_MIN = -32    # exp table domain [EXP_MIN, 0]
SILU_LIM = 32    # SiLU table domain [-SILU_LIM, SILU_LIM]
FL = 40          # ln table
MAX_POS = 2048


def exp_table(device=None):
    """e^x at FE bits for x = EXP_MIN .. 0 at step 2^-FA (2^17 + 1 entries; offline constant, float64 rounded
    once, src/bitexact/int8/consts.py:50-53)."""
    xs = torch.arange(EXP_MIN << FA, 1, dtype=torch.float64) / (1 << FA)
    t = torch.round(torch.exp(xs) * (1 << FE)).long()
    return t if device is None else t.to(device)


def silu_table(device=None):
    """SiLU(x) at FR bits for x in [-SILU_LIM, SILU_LIM] at step 2^-FA (2^18 + 1 entries; offline constant, float64
    rounded once, src/bitexact/int8/consts.py:79-80)."""
    xs = torch.arange(-SILU_LIM << FA, (SILU_LIM << FA) + 1, dtype=torch.float64) / (1 << FA)
    t = torch.round(xs / (1.0 + torch.exp(-xs)) * (1 << FR)).long()
    return t if device is None else t.to(device)
