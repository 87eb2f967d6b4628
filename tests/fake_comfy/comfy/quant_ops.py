"""comfy.quant_ops stand-in: QuantizedTensor and the layout registry."""
import torch

QUANT_ALGOS: dict = {}
_LAYOUTS: dict = {}


def register_layout_class(name, cls):
    _LAYOUTS[name] = cls


def get_layout_class(name):
    return _LAYOUTS[name]


class QuantizedTensor(torch.Tensor):
    """Wrapper tensor holding packed data (_qdata), a layout name and params."""

    @staticmethod
    def __new__(cls, qdata, layout_type, params):
        shape = tuple(params.orig_shape)
        t = torch.Tensor._make_wrapper_subclass(cls, shape, dtype=params.orig_dtype, device=qdata.device,
                                                requires_grad=False)
        t._qdata = qdata
        t._layout_type = layout_type
        t._params = params
        return t

    def __init__(self, qdata, layout_type, params):
        pass

    def __repr__(self):
        return f"QuantizedTensor({self._layout_type}, qdata={tuple(self._qdata.shape)})"

    def dequantize(self):
        return get_layout_class(self._layout_type).dequantize(self._qdata, self._params)

    @classmethod
    def __torch_dispatch__(cls, func, types, args=(), kwargs=None):
        kwargs = kwargs or {}
        name = func.overloadpacket.__name__
        if name in ("detach", "alias"):
            src = args[0]
            return QuantizedTensor(src._qdata, src._layout_type, src._params)
        if name == "_to_copy":
            src = args[0]
            dev = kwargs.get("device", None)
            if dev is None or dev == src._qdata.device:
                return QuantizedTensor(src._qdata, src._layout_type, src._params)
            import dataclasses

            p = src._params
            moved = {f.name: (getattr(p, f.name).to(dev) if isinstance(getattr(p, f.name), torch.Tensor)
                              else getattr(p, f.name)) for f in dataclasses.fields(p)}
            return QuantizedTensor(src._qdata.to(dev), src._layout_type, type(p)(**moved))
        raise NotImplementedError(f"QuantizedTensor stand-in does not implement {name}")
