"""Fixed DeepSeek-V3/R1 MoE geometry (kernels/moe.cu:41-53, reference/moe_ref.py:27-46)."""

H = 7168
I_DIM = 2048
E_GLOBAL = 256
E_LOCAL = 32
N_GROUP = 8
GROUP_SIZE = E_GLOBAL // N_GROUP
TOP_K = 8
TOPK_GROUP = 4
BLOCK = 128
H_BLOCKS = H // BLOCK            # 56
I_BLOCKS = I_DIM // BLOCK        # 16
G1_BLOCKS = 2 * I_DIM // BLOCK   # 32
MAX_E_LOCAL = 32
# Largest T served by the decode (weight-streaming) GEMMs; above it the
# prefill tile kernels run (csrc/common.h DECODE_MAX_T).
DECODE_MAX_T = 128

# Packed operand layouts (int32 views, 16 bytes per lane half):
#   W13: [E, nb=16, kb=56, tile=16, half=2, lane=64, 4]
#   W2 : [E, hb=56, kb=16, tile=8,  half=2, lane=64, 4]
W13_PACKED_SHAPE = (I_BLOCKS, H_BLOCKS, 16, 2, 64, 4)
W2_PACKED_SHAPE = (H_BLOCKS, I_BLOCKS, 8, 2, 64, 4)

# Algorithmic work per routed (token, local expert) pair: GEMM1 2*H*2I plus
# GEMM2 2*I*H (bench/bench_moe.py:29-32).
FLOPS_PER_ROUTE = 2 * H * (2 * I_DIM) + 2 * I_DIM * H
# Bytes per hit expert: W13 + W2 fp8 and their fp32 scales.
BYTES_PER_EXPERT = 2 * I_DIM * H + H * I_DIM + (G1_BLOCKS * H_BLOCKS + H_BLOCKS * I_BLOCKS) * 4
# Bytes per token: hidden fp8 + its scales + logits + bf16 output.
BYTES_PER_TOKEN = H + H_BLOCKS * 4 + E_GLOBAL * 4 + H * 2
BYTES_FIXED = E_GLOBAL * 2  # bias (bf16 at the surface)
