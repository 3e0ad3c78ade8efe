"""sparda — MI355X (gfx950) kernels for SparDA's forecast-guided block-sparse
attention, reached through the C ABI of libsparda.so (include/sparda.h)."""

from ._lib import (BF16, F32, FETCH_DMA, FETCH_KERNEL, ROUTE_ABSOLUTE, ROUTE_REFERENCE, SEL_DENSE, SEL_WINDOW_DECODE,
                   SEL_WINDOW_PREFILL, TOPK_AUTO, TOPK_ROWS, TOPK_WAVE, SpardaArgumentError,
                   SpardaError, load)
from .ops import (DecodeWorkspace, OffloadArena, append_at, block_sums, compress, decode, decode_at,
                  decode_selected, decode_sums, decode_workspace_bytes, default_scale, ffn_decode, gather_blocks, prefill,
                  prefill_chunked, prefill_masked, prefill_routed, produce,
                  norm_gemv, rows_residual,
                  require_device, route, select_chunked, select_decode, select_decode_at, select_fixed, status,
                  STATUS_PREFILL_WAIT_TIMEOUT, teacher_block_mass, topk_scores)

__all__ = [
    "BF16", "F32", "FETCH_DMA", "FETCH_KERNEL", "ROUTE_ABSOLUTE", "ROUTE_REFERENCE", "SEL_DENSE", "SEL_WINDOW_DECODE",
    "SEL_WINDOW_PREFILL", "TOPK_AUTO", "TOPK_ROWS", "TOPK_WAVE", "SpardaArgumentError", "SpardaError",
    "load", "DecodeWorkspace", "compress", "decode", "decode_workspace_bytes", "default_scale",
    "gather_blocks", "prefill", "prefill_chunked", "prefill_masked", "prefill_routed", "require_device", "route", "select_chunked",
    "select_fixed", "topk_scores",
    "OffloadArena", "decode_selected", "select_decode", "block_sums", "produce", "teacher_block_mass",
    "append_at", "select_decode_at", "decode_at", "ffn_decode", "decode_sums", "rows_residual", "norm_gemv",
    "status", "STATUS_PREFILL_WAIT_TIMEOUT",
]
