"""comfy.weight_adapter stand-in: the LoRA adapter object."""


class WeightAdapterBase:
    name = "base"


class LoRAAdapter(WeightAdapterBase):
    name = "lora"

    def __init__(self, weights):
        self.weights = weights
