"""SDXL-UNet layer shapes of the reference's benchmark configurations, shared
by bench.py and the GPU configuration tests.

Config 4: every SDXL-UNet Linear and 1x1 weight,
((out, in), count, tokens M), per notebook/src/sdxl_fit_smoketest.py:55-69 as
tabulated for this build.  Tokens per layer at batch 4 of a 128 x 128 latent,
realistic per level: 1280-channel layers at 32 x 32 (M 4096), 640-channel at
64 x 64 (M 16384), 320-channel at 128 x 128 (M 65536), cross-attention k/v on
77 x 4 text tokens (M 308), time/label embeddings on M 4.

Config 3: the linear shapes (out N, in K, tokens M) at batch 2
-- attention q/k/v/out, GEGLU in and out, the north-star shape, the
640-channel set on 4096 x 2 tokens, cross-attention k/v on 77 x 2 tokens.
"""
SDXL_LINEAR = [((10240, 1280), 60, 4096), ((1280, 1280), 381, 4096), ((1280, 5120), 60, 4096),
               ((1280, 2048), 120, 308), ((5120, 640), 10, 16384), ((640, 640), 70, 16384),
               ((640, 2048), 20, 308), ((640, 2560), 10, 16384), ((640, 1280), 5, 4),
               ((1280, 2816), 1, 4), ((320, 1280), 5, 4), ((1280, 320), 1, 4)]
SDXL_1X1 = [((1280, 2560), 2, 4096), ((1280, 1920), 1, 4096), ((640, 1920), 1, 16384),
            ((1280, 640), 1, 4096), ((640, 1280), 1, 16384), ((640, 960), 1, 16384),
            ((320, 640), 2, 65536), ((320, 960), 1, 65536), ((640, 320), 1, 16384)]

CONFIG3 = [(1280, 1280, 2048), (10240, 1280, 2048), (1280, 5120, 2048), (5120, 1280, 2048),
           (640, 640, 8192), (5120, 640, 8192), (640, 2560, 8192), (1280, 2048, 154)]
