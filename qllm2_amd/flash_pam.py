"""Drop-in for v11/flash_pam.py on the HIP scan.

flash_pam_chunked_head keeps the reference signature and return values
(v11/flash_pam.py:56-152): queries NOT pre-scaled (scaled by head_dim**-0.5
inside), keys/protected_values [B,H,T,d,2], decay_gamma [B,H,T]; returns
(output [B,H,T,d,2], memory_state [B,H,d,d,2]).  The whole chunk loop,
including the sequential state carry, runs in the qpam_scan_fwd kernels;
the backward runs in qpam_scan_bwd.

Ragged tail: the reference pads gamma with 1 to a chunk multiple, which
multiplies the final state by (1 + 1e-6)^pad (the padded log-decay is
log(1 + 1e-6) > 0); the kernel handles the ragged chunk without padding, so
its final state equals V11PAMLayer._forward_chunked_head's.  Outputs are
identical either way.
"""

import torch

from . import _reference
from .pam_scan import pam_scan_interleaved
from .triton_kernels import fused_decay_matrix

__all__ = ["flash_pam_chunked_head", "_chunk_decay_matrices"]


def _chunk_decay_matrices(decay_gamma_batch, chunk_len):
    """[N, C] -> (decay_matrix [N,C,C], cumulative_decay [N,C], total_decay [N],
    decay_last [N,C]) as v11/flash_pam.py:32-53.  The matrix comes from the
    HIP decay-matrix kernel; bf16/fp16 gamma is computed in fp32."""
    if not decay_gamma_batch.is_cuda:
        return _reference.on_cpu("flash_pam._chunk_decay_matrices", "_chunk_decay_matrices", decay_gamma_batch,
                                 chunk_len)
    compute = torch.float32 if decay_gamma_batch.dtype in (torch.bfloat16, torch.float16) else decay_gamma_batch.dtype
    g = decay_gamma_batch.to(compute)
    d_mat = fused_decay_matrix(g, chunk_len)
    cum = torch.exp(torch.cumsum(torch.log(g + 1e-6), dim=-1))
    return d_mat, cum, cum[:, -1], d_mat[:, -1, :]


def flash_pam_chunked_head(queries, keys, protected_values, decay_gamma, head_dim, chunk_size):
    """Chunk-parallel PAM scan, head-scalar decay (v11/flash_pam.py:56-152)."""
    if not queries.is_cuda:
        return _reference.on_cpu("flash_pam.flash_pam_chunked_head", "flash_pam_chunked_head", queries, keys,
                                 protected_values, decay_gamma, head_dim, chunk_size)
    y, s = pam_scan_interleaved(queries, keys, protected_values, decay_gamma.unsqueeze(0), head_dim, chunk_size)
    return y, s[0]
