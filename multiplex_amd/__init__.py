"""multiplex_amd: MI355X-native Gated DeltaNet hot path of wang1ang/multiplex.

The public functions mirror mlx-lm's ``mlx_lm.models.gated_delta`` module
(which multiplex calls from ``multiplex/kernel/dflash.py:372-374``) on
PyTorch-ROCm tensors, backed by hand-written gfx950 HIP kernels in
``libgdn.so`` (C ABI: ``include/gdn.h``).
"""

from .gated_delta import (
    CHUNK_MIN_TOKENS,
    chunk_workspace_bytes,
    compute_beta,
    compute_g,
    gated_delta_commit,
    gated_delta_commit_verify,
    gated_delta_kernel,
    gated_delta_ops,
    gated_delta_update,
    gated_delta_verify,
    prepare_chunked,
    prepare_recurrent,
)
from .conv import (conv_chunk_workspace_bytes, conv_state_commit, gdn_conv_chunked, gdn_conv_prologue,
                   prepare_conv_chunked, prepare_conv_prologue)
from .cache import ArraysCache, clone_ssm, merge_layer, restore_ssm, restore_ssm_snapshot, snapshot_ssm
from .state_pool import PooledBatch, StatePool
from . import prefix_state
from .epilogue import gated_rms_norm, prepare_gated_rms_norm
from .linear import DecodeWorkspace, gated_norm_linear_decode, linear_decode
from .mixer import GatedDeltaNet, commit_verified
from .mixed_step import MixedStep
from .attention import Attention, AttentionArgs, DecoderLayer, KVCache, MTPHead

__all__ = [
    "Attention",
    "AttentionArgs",
    "DecoderLayer",
    "KVCache",
    "MTPHead",
    "ArraysCache",
    "DecodeWorkspace",
    "GatedDeltaNet",
    "MixedStep",
    "PooledBatch",
    "StatePool",
    "clone_ssm",
    "commit_verified",
    "gated_rms_norm",
    "prepare_gated_rms_norm",
    "merge_layer",
    "restore_ssm",
    "restore_ssm_snapshot",
    "snapshot_ssm",
    "CHUNK_MIN_TOKENS",
    "chunk_workspace_bytes",
    "compute_beta",
    "compute_g",
    "conv_chunk_workspace_bytes",
    "conv_state_commit",
    "gdn_conv_chunked",
    "gated_delta_commit",
    "gated_delta_commit_verify",
    "gated_delta_kernel",
    "gated_delta_ops",
    "gated_delta_update",
    "gated_delta_verify",
    "gdn_conv_prologue",
    "gated_norm_linear_decode",
    "linear_decode",
    "prepare_chunked",
    "prepare_conv_chunked",
    "prepare_conv_prologue",
    "prepare_recurrent",
]
