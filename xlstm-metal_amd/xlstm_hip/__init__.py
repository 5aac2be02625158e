"""xlstm_hip — MI355X (gfx950) mLSTM/sLSTM kernel backend.

Drop-in for the torch-native kernel API of MLXPorts/xLSTM-metal: chunkwise
mLSTM prefill and its custom backward, recurrent decode step and sequence, sLSTM step and sequence,
the sLSTM layer's causal conv1d + SiLU and per-head GroupNorm, the mLSTM
output cell's multi-head RMSNorm x sigmoid(o), soft_cap and the logit
projection with its soft-cap epilogue,
each a ``torch.library`` op (``xlstm_hip::*``) calling hand-written HIP
kernels in ``lib/libxlstm_hip.so`` through a C-ABI.
"""

from . import _lib
from .backend import (
    available_kernels, get_mlstm_kernel, get_mlstm_sequence_kernel, get_mlstm_step_kernel, mLSTMBackend,
    mLSTMBackendConfig, wrap_chunkwise__arbitrary_sequence_length, wrap_chunkwise__pad_zeros,
)
from .chunkwise import mlstm_chunkwise, mlstm_chunkwise__native_autograd, mlstm_chunkwise__native_custbw
from .ops import chunkwise_algorithm
from .mlstm_layers import (
    MultiHeadLayerNorm, MultiHeadRMSNorm, gate_proj_softcap, mh_rmsnorm_gate, mLSTMOutputCell, mLSTMProjectionCell,
)
from .recurrent import (
    mLSTMRecurrentKernelCell, mlstm_recurrent_sequence__native_fw, mlstm_recurrent_step_,
    mlstm_recurrent_step__native, mlstm_recurrent_step__native_fw,
)
from .slstm import sLSTMStepwiseKernelCell, slstm_sequence, slstm_step, slstm_step_pytorch
from .slstm_layers import CausalConv1d, causal_conv1d, group_norm, sLSTMOutputCell, sLSTMProjectionCell
from .soft_cap import SoftCapCell, lm_head_softcap, soft_cap

LIB_PATH = _lib.LIB_PATH


def load_library():
    """Loads libxlstm_hip.so (raises RuntimeError if it has not been built)."""
    return _lib.load()


__all__ = [
    "mlstm_chunkwise", "mlstm_chunkwise__native_autograd", "mlstm_chunkwise__native_custbw",
    "chunkwise_algorithm", "mlstm_recurrent_step__native",
    "mlstm_recurrent_step__native_fw", "mlstm_recurrent_step_", "mlstm_recurrent_sequence__native_fw",
    "mLSTMRecurrentKernelCell",
    "slstm_step", "slstm_step_pytorch", "slstm_sequence", "sLSTMStepwiseKernelCell", "soft_cap", "SoftCapCell",
    "lm_head_softcap",
    "causal_conv1d", "group_norm", "CausalConv1d", "sLSTMProjectionCell", "sLSTMOutputCell",
    "mh_rmsnorm_gate", "MultiHeadRMSNorm", "MultiHeadLayerNorm", "mLSTMOutputCell", "gate_proj_softcap",
    "mLSTMProjectionCell",
    "get_mlstm_kernel", "get_mlstm_step_kernel", "get_mlstm_sequence_kernel", "available_kernels",
    "wrap_chunkwise__arbitrary_sequence_length", "wrap_chunkwise__pad_zeros", "mLSTMBackendConfig",
    "mLSTMBackend", "load_library", "LIB_PATH",
]
