// mia_internal.h — host-side declarations shared between the C-ABI layer
// (abi.hip) and the kernel translation units.  Not part of the public ABI.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <string>

#include "mia_attn.h"

namespace mia {

// Records `msg` as the calling thread's last error and returns `code`.
int set_error(int code, const std::string &msg);

// Checks a HIP call made while launching; converts failures to
// MIA_ERR_RUNTIME with the HIP error string.
int check_hip(hipError_t err, const char *what);

// Kernel launchers (each defined next to its kernels).  They assume the
// arguments were validated by the ABI layer.
int launch_kv_write(const mia_kv_write_args &a, hipStream_t s);
int launch_gather(const mia_gather_args &a, hipStream_t s);
int launch_decode_mask(const mia_mask_args &a, hipStream_t s);
int launch_slot_mapping(const mia_slot_mapping_args &a, hipStream_t s);
int launch_remap_null(const int32_t *in, int32_t *out, int64_t n,
                      int32_t null_block, hipStream_t s);
int launch_swa_trim(const mia_swa_trim_args &a, hipStream_t s);
int launch_packed_k(const mia_packed_k_args &a, hipStream_t s);
int launch_scatter_rows(const mia_scatter_rows_args &a, hipStream_t s);
int launch_stage_rows(const mia_stage_args &a, hipStream_t s);
int launch_qkv_epilogue(const mia_qkv_epilogue_args &a, hipStream_t s);
int launch_row_norm(const mia_row_norm_args &a, hipStream_t s);

// Paged decode: split-K plan shared by the workspace query and the launch.
struct DecodePlan {
  int split_tokens;  // min_tiles * 32
  int min_tiles;     // shortest tile range of a streaming wave
  int num_splits;    // partial slots per (row, kv head)
  int ncols;         // columns (query token x head of a GQA group) per launch
  int col_groups;    // launches over column groups
  int grid;          // workgroups of the persistent split-K kernel
  int one_pass;      // short tables: one wave per segment, no combine launch
  size_t ws_bytes;   // workspace bytes
};
DecodePlan plan_decode(const mia_decode_args &a);
// Batch rows of one decode launch sequence at most (per-row tables of the
// persistent split kernel live in LDS); the ABI layer runs larger batches as
// consecutive row chunks.
constexpr int kDecodeMaxRows = 1024;
// Device address of the current device's static decode scratch
// (MIA_DECODE_NOALLOC_SCRATCH_BYTES), looked up once per device.
int decode_noalloc_scratch(void **ptr);
int launch_paged_decode(const mia_decode_args &a, const DecodePlan &p,
                        hipStream_t s);
// The active K/V rows of a decode call written to its write_slots by one
// cache-write launch (the batch's rows as one token sequence, t = b * S + s).
int launch_decode_scatter(const mia_decode_args &a, hipStream_t s);

// Paged prefill: split-K plan shared by the workspace query and the launch.
struct PrefillPlan {
  bool dma;          // bf16 / head_dim 128 kernel with the LDS copy ring
  int dma_waves;     // its waves per workgroup (8, or 4 for compact launches)
  int rows_wg;       // query rows per workgroup
  int rows_max;      // max_seqlen_q * G
  int nsplit;        // key chunks per row tile at most (1: no split)
  int ksplit;        // keys per chunk (0: chosen on the device)
  int slots;         // workgroups resident on the device at once
  size_t ws_bytes;   // workspace bytes (0 without split)
};
PrefillPlan plan_prefill(const mia_prefill_args &a);
int launch_paged_prefill(const mia_prefill_args &a, const PrefillPlan &p, hipStream_t s);

}  // namespace mia
