"""End-to-end block-diffusion generation on the HIP path: a random-init
Qwen2.5-layout model (model.py) and the static-KV sampler (sampler.py)."""
