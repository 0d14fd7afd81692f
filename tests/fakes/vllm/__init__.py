"""Minimal stand-in for the parts of vLLM the fp8_huffman plugin imports (test infrastructure only).

vLLM is not installed in this image; the classes below carry just the
behaviour the plugin relies on: LinearBase is an nn.Module, quantization
configs register by name, and a BasevLLMParameter is a frozen Parameter that
carries its weight_loader.
"""
