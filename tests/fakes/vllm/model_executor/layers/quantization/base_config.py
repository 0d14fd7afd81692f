"""Stand-ins for vllm.model_executor.layers.quantization.base_config."""


class QuantizeMethodBase:
    pass


class QuantizationConfig:
    def __init__(self):
        pass
