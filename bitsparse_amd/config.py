"""Format constants of the BitSparse path.

Mirrors reference lib_sparse/config.py:1-12.  The 64x64 tile shape is part of
the compressed format and is fixed: every kernel in csrc/ assumes it.
"""
# ReLU^2 activation scale k in y = k * relu(z)^2 (reference config.py:2)
RELU2_SCALE = 1

# tile shape (reference config.py:5-6)
BLOCK_M = 64
BLOCK_N = 64

# tiles per staging chunk of the packed 15/7-bit value stream (reference config.py:9)
_PACK_CHUNK_TILES = 2**16

# keep fp8 copies of GEMM operands for the backward (reference config.py:12)
CACHE_FP8_MATMUl = False

# dtype of the gradients MatmulFp8 returns: None = the fp8 dtype of the
# operand each gradient belongs to, as the reference does (fp8.py:107,112);
# torch.bfloat16 keeps them in bf16 (an addition, not in the reference)
FP8_GRAD_DTYPE = None
