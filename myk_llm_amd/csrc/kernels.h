// Host-side launchers of the gfx950 kernels (one translation unit per kernel family).
// Each returns the HIP status of its launch; argument checking happens in api.hip.
#pragma once

#include <hip/hip_runtime.h>

#include "../../include/mykfa.h"

namespace mykfa {

hipError_t launch_fwd(const mykfa_fwd_params& p, hipStream_t stream);

hipError_t launch_bwd_preprocess(const mykfa_bwd_params& p, hipStream_t stream);
hipError_t launch_bwd_dkdv(const mykfa_bwd_params& p, hipStream_t stream);
hipError_t launch_bwd_dq(const mykfa_bwd_params& p, hipStream_t stream);
// Backward through stored dS: bytes of dS one KV head's query heads take (0: no such path for
// this head_dim), and the launches (delta; per pass of kv_per_pass KV heads, dK/dV storing dS
// into ws, then dQ from it).
size_t bwd_ds_bytes_per_kv_head(const mykfa_bwd_params& p);
hipError_t launch_bwd_ds(const mykfa_bwd_params& p, void* ws, int kv_per_pass, hipStream_t stream);
// One half of it over every KV head at once: dK/dV storing dS (dq = false) or dQ from dS.
hipError_t launch_bwd_ds_half(const mykfa_bwd_params& p, void* ws, bool dq, hipStream_t stream);

// Split-K decode. The workspace holds, per (split, batch, head, query): D fp32 partial
// outputs, then one fp32 partial lse per (split, batch, head, query).
size_t decode_workspace_bytes(int batch, int num_heads, int seqlen_q, int head_dim, int num_splits);
int decode_default_splits(int batch, int num_heads, int num_kv_heads, int seqlen_q, int capacity);
hipError_t launch_decode_splitk(const mykfa_decode_params& p, int num_splits, void* ws, hipStream_t stream);
hipError_t launch_decode_merge(const mykfa_decode_params& p, int num_splits, const void* ws,
                               hipStream_t stream);
// This device's copy of the allocation-free decode's static scratch array (resolved once per
// device; MYKFA_DECODE_SCRATCH_BYTES long).
hipError_t decode_scratch(hipStream_t stream, void** ptr);

hipError_t launch_kv_append(const mykfa_kv_append_params& p, hipStream_t stream);

// Attention-block prologue (q/k RMSNorm + RoPE) and epilogue (output gate), block_io.hip.
// The backward's grid (bounded, so the weight-gradient partials have a fixed count) and the
// fp32 workspace holding one (2, head_dim) partial per workgroup.
int qk_prologue_bwd_blocks(int batch, int seqlen, int num_heads, int num_kv_heads, int head_dim);
size_t qk_prologue_bwd_workspace_bytes(int batch, int seqlen, int num_heads, int num_kv_heads, int head_dim);
hipError_t launch_qk_prologue_fwd(const mykfa_qk_prologue_params& p, hipStream_t stream);
hipError_t launch_qk_prologue_bwd(const mykfa_qk_prologue_bwd_params& p, void* ws, hipStream_t stream);
hipError_t launch_gate(const mykfa_gate_params& p, bool backward, hipStream_t stream);

// Cross-entropy rows of the fused linear + cross-entropy (fused_ce.hip).
hipError_t launch_ce_rows(const mykfa_ce_params& p, hipStream_t stream);

// Batched SYRK of Muon's Newton-Schulz iteration (syrk.hip).
hipError_t launch_syrk(const mykfa_syrk_params& p, hipStream_t stream);

}  // namespace mykfa
