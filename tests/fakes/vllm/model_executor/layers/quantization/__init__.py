"""Stand-in for vllm.model_executor.layers.quantization: a name -> config registry."""
REGISTRY = {}


def register_quantization_config(name):
    def deco(cls):
        REGISTRY[name] = cls
        return cls
    return deco
