"""Linear layers whose AWQ projections call the W4A16 HIP method: the call sites of the
reference's boundary (llmserve/layers/linear.py).

* ``LinearBase.apply_linear`` -> ``quant_method.apply(self, x)``   linear.py:54-57
* ``RowParallelLinear.forward`` -> ``quant_method.apply``           linear.py:228-236
* packed-output-dim weight loaders (merged gate/up, q/k/v)         linear.py:109-196, 217-226
* ``validate_awq_output_shards``                                   linear.py:14-21

Tensor parallelism follows the reference: AWQ layers require a world size of 1
(AWQLinearMethod.create_weights raises otherwise).  Rank and world size come from
torch.distributed when it is initialised, else (0, 1).
"""
from __future__ import annotations

import torch
import torch.distributed as dist
import torch.nn.functional as F
from torch import nn

from .quantization.awq import AWQLinearMethod, AWQRuntimeConfig


def divide(numerator: int, denominator: int) -> int:
    assert numerator % denominator == 0
    return numerator // denominator


def tp_rank() -> int:
    return dist.get_rank() if dist.is_available() and dist.is_initialized() else 0


def tp_world_size() -> int:
    return dist.get_world_size() if dist.is_available() and dist.is_initialized() else 1


def validate_awq_output_shards(output_sizes: list[int], quant_config: AWQRuntimeConfig | None) -> None:
    if quant_config is None:
        return
    if any(size % quant_config.pack_factor for size in output_sizes):
        raise ValueError("each AWQ output shard must be divisible by pack_factor")


class LinearBase(nn.Module):

    def __init__(self, input_size: int, output_size: int, bias: bool = False, tp_dim: int | None = None,
                 quant_config: AWQRuntimeConfig | None = None):
        super().__init__()
        self.tp_dim = tp_dim
        self.tp_rank = tp_rank()
        self.tp_size = tp_world_size()
        self.quant_method = AWQLinearMethod(quant_config) if quant_config else None
        if self.quant_method is None:
            self.weight = nn.Parameter(torch.empty(output_size, input_size))
            self.weight.weight_loader = self.weight_loader
        else:
            if bias:
                raise ValueError("AWQ Linear bias is not supported")
            self.quant_method.create_weights(self, input_size, output_size)
            for param in (self.qweight, self.qzeros, self.scales):
                param.weight_loader = self.weight_loader
        if bias:
            self.bias = nn.Parameter(torch.empty(output_size))
            self.bias.weight_loader = self.weight_loader
        else:
            self.register_parameter("bias", None)

    def apply_linear(self, x: torch.Tensor) -> torch.Tensor:
        if self.quant_method is not None:
            return self.quant_method.apply(self, x)
        return F.linear(x, self.weight, self.bias)

    @staticmethod
    def get_output_dim(param: nn.Parameter, default: int) -> int:
        return getattr(param, "output_dim", default)

    @staticmethod
    def get_packed_factor(param: nn.Parameter, dim: int) -> int:
        if getattr(param, "packed_dim", None) == dim:
            return getattr(param, "pack_factor")
        return 1

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        raise NotImplementedError


class ReplicatedLinear(LinearBase):

    def __init__(self, input_size: int, output_size: int, bias: bool = False,
                 quant_config: AWQRuntimeConfig | None = None):
        super().__init__(input_size, output_size, bias, quant_config=quant_config)

    def weight_loader(self, param: nn.Parameter, loaded_weight: torch.Tensor):
        param.data.copy_(loaded_weight)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        return self.apply_linear(x)


class ColumnParallelLinear(LinearBase):

    def __init__(self, input_size: int, output_size: int, bias: bool = False,
                 quant_config: AWQRuntimeConfig | None = None):
        super().__init__(input_size, divide(output_size, tp_world_size()), bias, 0, quant_config)

    def weight_loader(self, param: nn.Parameter, loaded_weight: torch.Tensor):
        output_dim = self.get_output_dim(param, self.tp_dim)
        shard_size = param.data.size(output_dim)
        loaded_weight = loaded_weight.narrow(output_dim, self.tp_rank * shard_size, shard_size)
        param.data.copy_(loaded_weight)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        return self.apply_linear(x)

    def forward_rmsnorm(self, norm: nn.Module, x: torch.Tensor, residual: torch.Tensor | None = None):
        """``self(norm(x, residual))`` for an RMSNorm ``norm`` (its ``weight`` and ``eps``) in
        front of this projection -- input_layernorm then qkv_proj (qwen3.py:166-169) -- as
        one library call; returns ``(y, new residual)``.  Without a residual (the first
        layer) the new residual is ``x`` itself, as qwen3.py:166-167 sets it."""
        return self._rmsnorm_apply(norm, x, residual, silu_mul=False)

    def forward_rmsnorm_stats(self, norm: nn.Module, inp) -> torch.Tensor:
        """``self(norm(h, residual))`` where the producer before the norm already added the
        residual and left its row statistics (``NormInput`` of
        RowParallelLinear.forward_residual_stats): the norm's scaling and this projection in
        one decode kernel; the new residual came from the producer."""
        return self._rmsnorm_stats_apply(norm, inp, silu_mul=False)

    def _rmsnorm_stats_apply(self, norm: nn.Module, inp, silu_mul: bool):
        if self.quant_method is None or not hasattr(self.quant_method, "apply_rmsnorm_stats"):
            raise ValueError("the fused RMSNorm statistics are implemented for the AWQ HIP backend only")
        return self.quant_method.apply_rmsnorm_stats(self, inp, norm.weight, norm.eps, silu_mul=silu_mul)

    def _rmsnorm_apply(self, norm: nn.Module, x: torch.Tensor, residual: torch.Tensor | None, silu_mul: bool):
        if self.quant_method is None or not hasattr(self.quant_method, "apply_rmsnorm"):
            raise ValueError("the fused RMSNorm prologue is implemented for the AWQ HIP backend only")
        return self.quant_method.apply_rmsnorm(self, x, residual, norm.weight, norm.eps, silu_mul=silu_mul)


class MergedColumnParallelLinear(ColumnParallelLinear):

    def __init__(self, input_size: int, output_sizes: list[int], bias: bool = False,
                 quant_config: AWQRuntimeConfig | None = None):
        validate_awq_output_shards(output_sizes, quant_config)
        self.output_sizes = output_sizes
        super().__init__(input_size, sum(output_sizes), bias, quant_config)
        for param in self.parameters(recurse=False):
            param.expected_shard_ids = tuple(range(len(output_sizes)))

    def weight_loader(self, param: nn.Parameter, loaded_weight: torch.Tensor, loaded_shard_id: int):
        output_dim = self.get_output_dim(param, self.tp_dim)
        pack_factor = self.get_packed_factor(param, output_dim)
        shard_offset = sum(self.output_sizes[:loaded_shard_id]) // self.tp_size // pack_factor
        shard_size = self.output_sizes[loaded_shard_id] // self.tp_size // pack_factor
        param_data = param.data.narrow(output_dim, shard_offset, shard_size)
        loaded_weight = loaded_weight.chunk(self.tp_size, output_dim)[self.tp_rank]
        param_data.copy_(loaded_weight)

    def forward_silu_and_mul(self, x: torch.Tensor) -> torch.Tensor:
        """``SiluAndMul()(self(x))`` for a [gate, up] layer of two equal shards
        (qwen3.py:126-130 with activation.py:8-11), fused into the AWQ GEMM epilogue: the
        [M, 2 I] intermediate is never written."""
        if len(self.output_sizes) != 2 or self.output_sizes[0] != self.output_sizes[1]:
            raise ValueError("fused SiLU * up needs exactly two equal output shards (gate, up)")
        if self.quant_method is None or not hasattr(self.quant_method, "apply_silu_and_mul"):
            raise ValueError("fused SiLU * up is implemented for the AWQ HIP backend only")
        return self.quant_method.apply_silu_and_mul(self, x)

    def forward_rmsnorm_silu_and_mul(self, norm: nn.Module, x: torch.Tensor, residual: torch.Tensor | None = None):
        """``SiluAndMul()(self(norm(x, residual)))`` -- post_attention_layernorm then the MLP's
        gate_up and activation (qwen3.py:172-173, 126-130) -- as one library call; returns
        ``(y, new residual)`` (``x`` itself when no residual is given)."""
        if len(self.output_sizes) != 2 or self.output_sizes[0] != self.output_sizes[1]:
            raise ValueError("fused SiLU * up needs exactly two equal output shards (gate, up)")
        return self._rmsnorm_apply(norm, x, residual, silu_mul=True)

    def forward_rmsnorm_stats_silu_and_mul(self, norm: nn.Module, inp) -> torch.Tensor:
        """``SiluAndMul()(self(norm(h, residual)))`` from a producer's ``NormInput`` (see
        ColumnParallelLinear.forward_rmsnorm_stats)."""
        if len(self.output_sizes) != 2 or self.output_sizes[0] != self.output_sizes[1]:
            raise ValueError("fused SiLU * up needs exactly two equal output shards (gate, up)")
        return self._rmsnorm_stats_apply(norm, inp, silu_mul=True)


class QKVParallelLinear(ColumnParallelLinear):

    def __init__(self, hidden_size: int, head_size: int, total_num_heads: int,
                 total_num_kv_heads: int | None = None, bias: bool = False,
                 quant_config: AWQRuntimeConfig | None = None):
        tp_size = tp_world_size()
        total_num_kv_heads = total_num_kv_heads or total_num_heads
        self.head_size = head_size
        self.num_heads = divide(total_num_heads, tp_size)
        self.num_kv_heads = divide(total_num_kv_heads, tp_size)
        validate_awq_output_shards(
            [total_num_heads * head_size, total_num_kv_heads * head_size, total_num_kv_heads * head_size],
            quant_config)
        output_size = (total_num_heads + 2 * total_num_kv_heads) * head_size
        super().__init__(hidden_size, output_size, bias, quant_config)
        for param in self.parameters(recurse=False):
            param.expected_shard_ids = ("q", "k", "v")

    def weight_loader(self, param: nn.Parameter, loaded_weight: torch.Tensor, loaded_shard_id: str):
        assert loaded_shard_id in ("q", "k", "v")
        output_dim = self.get_output_dim(param, self.tp_dim)
        pack_factor = self.get_packed_factor(param, output_dim)
        q_size = self.num_heads * self.head_size
        kv_size = self.num_kv_heads * self.head_size
        if loaded_shard_id == "q":
            shard_offset, shard_size = 0, q_size
        elif loaded_shard_id == "k":
            shard_offset, shard_size = q_size, kv_size
        else:
            shard_offset, shard_size = q_size + kv_size, kv_size
        param_data = param.data.narrow(output_dim, shard_offset // pack_factor, shard_size // pack_factor)
        loaded_weight = loaded_weight.chunk(self.tp_size, output_dim)[self.tp_rank]
        param_data.copy_(loaded_weight)


class RowParallelLinear(LinearBase):

    def __init__(self, input_size: int, output_size: int, bias: bool = False,
                 quant_config: AWQRuntimeConfig | None = None):
        super().__init__(divide(input_size, tp_world_size()), output_size, bias, 1, quant_config)

    def weight_loader(self, param: nn.Parameter, loaded_weight: torch.Tensor):
        param_data = param.data
        if param_data.ndim == 1:
            param_data.copy_(loaded_weight)
            return
        input_dim = getattr(param, "input_dim", self.tp_dim)
        shard_size = param_data.size(input_dim)
        loaded_weight = loaded_weight.narrow(input_dim, self.tp_rank * shard_size, shard_size)
        param_data.copy_(loaded_weight)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        if self.quant_method is None:
            bias = self.bias if self.tp_rank == 0 else None
            y = F.linear(x, self.weight, bias)
        else:
            y = self.quant_method.apply(self, x)
        if self.tp_size > 1:
            dist.all_reduce(y)
        return y

    def forward_residual(self, x: torch.Tensor, residual: torch.Tensor,
                         out: torch.Tensor | None = None) -> torch.Tensor:
        """The new residual ``bf16(self(x).float() + residual.float())`` of the next
        add_rms_forward (layernorm.py:35-36, after O and down in qwen3.py:170-174) with the
        add in the AWQ GEMM epilogue; ``out`` may be ``residual`` for an in-place update.
        The RMSNorm itself stays with the norm layer."""
        if self.quant_method is None or not hasattr(self.quant_method, "apply_residual"):
            raise ValueError("the fused residual add is implemented for the AWQ HIP backend only")
        if self.tp_size > 1:
            raise ValueError("the fused residual add needs a tensor-parallel world size of 1")
        return self.quant_method.apply_residual(self, x, residual, out=out)

    def forward_residual_stats(self, x: torch.Tensor, residual: torch.Tensor,
                               residual_out: torch.Tensor | None = None):
        """At decode sizes (packed M <= 8; faster than a separate norm launch up to M = 4):
        this projection, the residual add of the next add_rms_forward and that norm's row
        statistics in the GEMM epilogue, so that the norm needs no launch of its own; returns
        ``(NormInput, new residual)`` for the next layer's forward_rmsnorm_stats.
        ``residual_out`` may be ``residual`` (in place)."""
        if self.quant_method is None or not hasattr(self.quant_method, "apply_residual_stats"):
            raise ValueError("the fused RMSNorm statistics are implemented for the AWQ HIP backend only")
        if self.tp_size > 1:
            raise ValueError("the fused residual add needs a tensor-parallel world size of 1")
        return self.quant_method.apply_residual_stats(self, x, residual, residual_out=residual_out)
