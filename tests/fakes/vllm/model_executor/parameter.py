"""Stand-in for vllm.model_executor.parameter.BasevLLMParameter."""
import torch


class BasevLLMParameter(torch.nn.Parameter):
    def __new__(cls, data, **kwargs):
        return super().__new__(cls, data=data, requires_grad=False)

    def __init__(self, data, weight_loader=None):
        self._weight_loader = weight_loader

    @property
    def weight_loader(self):
        return self._weight_loader
