"""pararnn_amd — MI355X-native fused Newton + parallel scan for ParaRNN cells.

Drop-in for the reference's ``newton_apply`` / ``NewtonConfig`` path on
``ParaSLSTM(mix='diag')`` (per-channel 4x4 Jacobian) and ``ParaGRU(mix='head')``
(block-diagonal 64x64 Jacobian).  The solve runs hand-written HIP kernels for
gfx950 through a C ABI (``include/pararnn_amd.h``) loaded with ctypes; the
ops are registered as ``torch.library`` custom ops under the reference's
names (``pararnn::newton_slstm_fused``, ``pararnn::newton_gru_head_fused``).
"""

from pararnn_amd.cells import ParaGRU, ParaSLSTM
from pararnn_amd.decode import can_decode_step, decode_step, decode_wx
from pararnn_amd.config import (
    LIBRARY_NEWTON_ITERS,
    NewtonConfig,
    NewtonDivergenceError,
    NewtonStats,
    compile_safe_config,
)
from pararnn_amd.newton import (
    auto_newton_iters,
    fused_newton,
    newton_apply,
    slstm_auto_picard,
    slstm_picard_next,
)
from pararnn_amd.layers import ParaRNN
from pararnn_amd.ops import newton_gru_head_fused, newton_slstm_fused, slstm_init_fused
from pararnn_amd.sequential import sequential_apply
from pararnn_amd.verify import (
    AgreementError,
    AgreementReport,
    default_agreement_atol,
    verify_agreement,
)

__version__ = "0.1.0"

__all__ = [
    "AgreementError",
    "AgreementReport",
    "LIBRARY_NEWTON_ITERS",
    "NewtonConfig",
    "NewtonDivergenceError",
    "NewtonStats",
    "ParaGRU",
    "ParaRNN",
    "ParaSLSTM",
    "auto_newton_iters",
    "can_decode_step",
    "decode_step",
    "decode_wx",
    "compile_safe_config",
    "default_agreement_atol",
    "fused_newton",
    "newton_apply",
    "newton_gru_head_fused",
    "newton_slstm_fused",
    "sequential_apply",
    "slstm_auto_picard",
    "slstm_init_fused",
    "slstm_picard_next",
    "verify_agreement",
]
