"""yalm_amd: MI355X-native fp16 batch-1 decode path for yalm-format (Llama/Mistral) models.

The product is two native libraries built in-tree:
  libyalm_hip.so   -- gfx950 HIP kernels behind the C-ABI in include/yalm_hip.h
  libyalm_host.so  -- C++ host mirror of the reference Model/InferenceState API (Device::HIP),
                      the .yalm codec, sampler, tokenizer and synthetic-model writer
plus the `yalm` command-line binary. `yalm_amd.hip` and `yalm_amd.host` are thin ctypes bindings.
"""
