"""comfy.ops stand-in: CastWeightBiasOp / manual_cast and the cast hooks."""
import torch
import torch.nn.functional as F

CAST_CALLS = []


def cast_bias_weight(s, input=None, dtype=None, device=None, bias_dtype=None, offloadable=False):
    """Moves weight and bias to `device` (a QuantizedTensor stays quantized)."""
    weight = s.weight
    bias = s.bias
    if device is not None:
        weight = weight.to(device) if not hasattr(weight, "_qdata") else weight
        bias = bias.to(device=device, dtype=bias_dtype) if bias is not None else None
    CAST_CALLS.append(("cast", id(s)))
    if offloadable:
        return weight, bias, None
    return weight, bias


def uncast_bias_weight(s, weight, bias, offload_stream):
    CAST_CALLS.append(("uncast", id(s)))


class CastWeightBiasOp:
    comfy_cast_weights = False
    weight_function = []
    bias_function = []


class disable_weight_init:
    class Linear(torch.nn.Linear, CastWeightBiasOp):
        def reset_parameters(self):
            return None

        def forward(self, input):
            weight, bias = self.weight, self.bias
            return F.linear(input, weight.to(input.dtype), None if bias is None else bias.to(input.dtype))

    class GroupNorm(torch.nn.GroupNorm, CastWeightBiasOp):
        pass

    class LayerNorm(torch.nn.LayerNorm, CastWeightBiasOp):
        pass

    class Conv2d(torch.nn.Conv2d, CastWeightBiasOp):
        pass

    class Conv3d(torch.nn.Conv3d, CastWeightBiasOp):
        pass

    class ConvTranspose2d(torch.nn.ConvTranspose2d, CastWeightBiasOp):
        pass

    class Embedding(torch.nn.Embedding, CastWeightBiasOp):
        pass


class manual_cast(disable_weight_init):
    class Linear(disable_weight_init.Linear):
        pass

    class GroupNorm(disable_weight_init.GroupNorm):
        pass

    class LayerNorm(disable_weight_init.LayerNorm):
        pass

    class Conv2d(disable_weight_init.Conv2d):
        pass

    class Conv3d(disable_weight_init.Conv3d):
        pass

    class ConvTranspose2d(disable_weight_init.ConvTranspose2d):
        pass

    class Embedding(disable_weight_init.Embedding):
        pass
