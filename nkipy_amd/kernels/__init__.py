"""NumPy kernels of the hot path, written the way NKIPy kernels are written:
plain NumPy functions that run on the CPU when called directly and are
traced onto the gfx950 kernels under ``trace`` / ``baremetal_jit`` /
``DeviceKernel``.  They follow the reference's example kernels (cited per
function) and the workloads of the backend's benchmark.
"""

from nkipy_amd.kernels.softmax import softmax_kernel, softmax_upcast_kernel  # noqa: F401
from nkipy_amd.kernels.rmsnorm import residual_rmsnorm_kernel, rmsnorm_kernel  # noqa: F401
from nkipy_amd.kernels.feedforward import (  # noqa: F401
    feedforward_bias_kernel, feedforward_kernel, linear_nt_kernel, swiglu_mlp_kernel,
)
from nkipy_amd.kernels.linear_attention import chunked_linear_attention_kernel  # noqa: F401
from nkipy_amd.kernels.decoder import (  # noqa: F401
    attention_block_fp8, causal_gqa_attention_kernel, llama_decoder_layer_fp8, mlp_block_fp8,
    qkv_rope_fp8, rope_kernel, rope_tables,
)
