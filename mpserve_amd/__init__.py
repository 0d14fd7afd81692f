"""mpserve_amd: MPServe's FP8 + Huffman-sidecar weight path on AMD MI355X (gfx950).

* ``mpserve_amd.mpserve_cuda`` — the reference's ``MPServe_cuda`` op surface
  (build + decode), over hand-written HIP kernels in ``libmpserve_amd.so``.
* ``mpserve_amd.decode.DecodePlan`` — one launch for many tensors.
* ``mpserve_amd.vllm_fp8_huffman`` — the vLLM ``fp8_huffman`` quantization method.
"""
__version__ = "0.1.0"
