"""MI355X-native (gfx950) NF4-LoRA projection path with causal-tuner's operator API.

Module layout follows the reference package (src/causal_tuner/): `kernels.linear`,
`kernels.nf4_cuda`, `kernels.mlp_cuda` and `modeling.lora` keep its names and signatures;
their device work runs in the hand-written HIP kernels of lib/libcausal_tuner_hip.so.
"""
