"""Stand-ins for vllm.model_executor.layers.linear."""
import torch


class LinearMethodBase:
    def create_weights(self, *args, **kwargs):
        raise NotImplementedError

    def apply(self, layer, x, bias=None):
        raise NotImplementedError

    def process_weights_after_loading(self, layer):
        return None


class UnquantizedLinearMethod(LinearMethodBase):
    def apply(self, layer, x, bias=None):
        out = torch.matmul(x, layer.weight.t())
        return out if bias is None else out + bias


class LinearBase(torch.nn.Module):
    """A linear layer shell: the plugin only needs isinstance() and attributes set by the test."""

    def __init__(self, prefix: str = ""):
        super().__init__()
        self.prefix = prefix
