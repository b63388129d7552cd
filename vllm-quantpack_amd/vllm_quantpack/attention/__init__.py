"""int4_per_token_head / k8v4_per_token_head KV-cache attention on gfx950 HIP kernels."""
