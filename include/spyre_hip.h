/*
 * spyre_hip.h -- C ABI of the MI355X (gfx950) stick-relayout and paged
 * decode-attention library (libspyre_hip.so).
 *
 * Plain pointers and sizes only.  Device pointers are HIP device addresses;
 * `stream` is a hipStream_t passed as void* (NULL = the default stream).
 * Every entry point is asynchronous on `stream` and never allocates or frees
 * device memory: the caller owns every buffer, including workspaces.
 *
 * Return codes: SPYRE_OK (0) or a negative SPYRE_E* code; the message of the
 * last failure on the calling thread is available from spyre_last_error().
 *
 * Reference paths below are relative to the torch-spyre repository root.
 */
#ifndef SPYRE_HIP_H
#define SPYRE_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define SPYRE_ABI_VERSION 1

#define SPYRE_OK 0
#define SPYRE_EINVAL (-1)      /* bad argument (shape, stride, pointer)      */
#define SPYRE_EUNSUPPORTED (-2) /* valid but not handled by a fast path       */
#define SPYRE_ENOSPC (-3)      /* workspace / output buffer too small         */
#define SPYRE_EHIP (-4)        /* a HIP runtime call failed                  */

#define SPYRE_MAX_RANK 8       /* device rank of a layout: host rank <= 6, +1 */
#define SPYRE_MAX_INFOS 64     /* loop nests per DMA description              */

/* Device data formats on this path; names follow the reference's DataFormats
 * (torch_spyre/csrc/module.cpp:295-316, torch_spyre/csrc/types_mapping.h:71-92). */
#define SPYRE_FMT_INVALID 0
#define SPYRE_FMT_SEN169_FP16 1
#define SPYRE_FMT_IEEE_FP32 2
#define SPYRE_FMT_IEEE_INT32 3

/* Host element types, numbered as c10::ScalarType. */
#define SPYRE_DT_INT32 3
#define SPYRE_DT_INT64 4
#define SPYRE_DT_FLOAT16 5
#define SPYRE_DT_FLOAT32 6
#define SPYRE_DT_BOOL 11
#define SPYRE_DT_BFLOAT16 15

/* One DMA loop nest (the reference's DataConversionStrideInfo,
 * torch_spyre/csrc/spyre_mem.cpp:320-352).  Lists are innermost loop first;
 * strides and offsets are in elements. */
typedef struct spyre_stride_info {
  int32_t rank;
  int32_t reserved;
  int64_t size[SPYRE_MAX_RANK];
  int64_t stride_src[SPYRE_MAX_RANK];
  int64_t stride_dst[SPYRE_MAX_RANK];
  int64_t offset_src;
  int64_t offset_dst;
} spyre_stride_info;

/* ---------------------------------------------------------------- misc -- */

int spyre_abi_version(void);
const char* spyre_last_error(void);

/* --------------------------------------- layout descriptor (host only) -- */

/* Device format of a host element type; SPYRE_FMT_INVALID if unsupported.
 * Replaces stringToDTDataFormatPair (torch_spyre/csrc/types_mapping.h:63-113)
 * as used by SpyreTensorLayout::init (torch_spyre/csrc/spyre_tensor_impl.cpp:141-144). */
int spyre_device_format(int scalar_type);

/* Elements per 128-byte stick of a device format, or -1.
 * Replaces spyre::elems_per_stick (torch_spyre/csrc/spyre_tensor_impl.cpp:33-40). */
int64_t spyre_elems_per_stick(int data_format);

/* SpyreTensorLayout(host_size, host_strides, dtype, dim_order) and, with
 * host_strides == NULL and dim_order == NULL, SpyreTensorLayout(host_size,
 * dtype).  dim_order may carry a trailing -1 (sparse layout).  Writes
 * device_rank entries to device_size/stride_map (capacity SPYRE_MAX_RANK).
 * Replaces SpyreTensorLayout::init (torch_spyre/csrc/spyre_tensor_impl.cpp:124-179,
 * bound at torch_spyre/csrc/module.cpp:229-232). */
int spyre_stl_init(const int64_t* host_size, int host_rank, const int64_t* host_strides,
                   int scalar_type, const int32_t* dim_order, int dim_order_len,
                   int64_t* device_size, int64_t* stride_map, int* device_rank,
                   int* data_format);

/* 128 bytes x product(device_size[:-1]).
 * Replaces get_device_size_in_bytes (torch_spyre/csrc/spyre_tensor_impl.cpp:286-292). */
uint64_t spyre_device_size_in_bytes(const int64_t* device_size, int device_rank);

/* DMA description of a host<->device relayout: the loop nests the reference
 * hands to its DMA engine.  sizes/dma_strides/cpu_strides have host_rank
 * entries.  Replaces get_device_stride_infos
 * (torch_spyre/csrc/spyre_mem.cpp:176-354, called from generate_dci :363-440). */
int spyre_dma_plan(const int64_t* sizes, const int64_t* dma_strides, const int64_t* cpu_strides,
                   int host_rank, int64_t storage_offset, const int64_t* device_size,
                   const int64_t* stride_map, int device_rank, int host2device,
                   spyre_stride_info* infos, int max_infos, int* n_infos);

/* Single loop nest moving a dense host tensor of host_size from device layout
 * A to device layout B (both exact: no padding, no broadcast), i.e. the
 * device-side restickify.  SPYRE_EUNSUPPORTED when the two tilings do not
 * nest (the caller then relayouts through a host-layout buffer).
 * Replaces the ReStickifyOpHBM program emitted for spyre::restickify
 * (torch_spyre/_inductor/customops.py:338-342, lowering.py:803-833,
 * codegen/superdsc.py:761-803). */
int spyre_restick_plan(const int64_t* host_size, int host_rank,
                       const int64_t* src_device_size, const int64_t* src_stride_map, int src_rank,
                       const int64_t* dst_device_size, const int64_t* dst_stride_map, int dst_rank,
                       spyre_stride_info* info);

/* --------------------------------------------------------- GPU kernels -- */

/* Executes DMA loop nests on the GPU: for every index tuple of every info,
 * dst[offset_dst + i.stride_dst] = src[offset_src + i.stride_src], moving raw
 * elem_bytes-sized elements (1, 2, 4 or 8; bit-exact).  Stick-preserving
 * nests run as 16-byte vector copies, stick-transposing nests as 8x8
 * register-transposed tiles.  Every nest is checked against src_bytes /
 * dst_bytes before anything is launched.  Replaces the DMA launch of
 * SpyreStream::copyAsyncImpl (torch_spyre/csrc/spyre_stream.cpp:190-210). */
int spyre_dma_copy(const void* src, size_t src_bytes, void* dst, size_t dst_bytes, int elem_bytes,
                   const spyre_stride_info* infos, int n_infos, void* stream);

/* Batched KV-cache append into the paged stick-layout cache (relayout on
 * write).  For every sequence b the new token goes to position
 * positions[b]: page block_table[b*bt_stride + positions[b]/page_size],
 * slot positions[b] % page_size; each table row holds pages_per_seq entries.
 *   k_new, v_new : [B, Hkv, D] fp16, row-major
 *   k_cache      : [num_pages, Hkv, D/64, page_size, 64] fp16 (sticks on D)
 *   v_cache      : [num_pages, Hkv, D, page_size]      fp16 (sticks on tokens)
 * Sequences with positions[b] < 0 are skipped; positions past the row and
 * page ids outside [0, num_pages) are dropped (never written).  Replaces the per-offset
 * spyre::overwrite programs (torch_spyre/_inductor/customops.py:260-308,
 * tests/inductor/test_overwrite.py) with one launch whose offsets are data. */
int spyre_kv_append_f16(const void* k_new, const void* v_new, void* k_cache, void* v_cache,
                        const int32_t* block_table, int64_t bt_stride, int64_t pages_per_seq,
                        const int32_t* positions, int B, int Hkv, int D, int page_size,
                        int64_t num_pages, void* stream);

/* Workspace bytes needed by spyre_paged_decode_attn_f16: fp32 chunk
 * partials, B * Hkv * ceil(max_context_len / (8 * split_tokens)) * g * (D + 2)
 * floats, then a 4-byte arrival flag per (sequence, KV head, chunk).  The
 * contents need no initialisation. */
size_t spyre_paged_decode_attn_workspace_bytes(int B, int Hq, int Hkv, int D, int max_context_len,
                                               int split_tokens);

/* Split-KV paged decode attention, one query token per sequence:
 *   out[b,h,:] = softmax(scale * q[b,h,:] . K[b,h/g,t,:]^T) V[b,h/g,t,:],
 *   t < context_lens[b], g = Hq / Hkv (GQA: q head h reads KV head h/g).
 *   q, out       : [B, Hq, D] fp16 row-major
 *   k_cache      : [num_pages, Hkv, D/64, page_size, 64] fp16 (sticks on D)
 *   v_cache      : [num_pages, Hkv, D, page_size]      fp16 (sticks on tokens)
 *   block_table  : int32, row b at block_table + b*bt_stride
 *   context_lens : int32 [B]; every context_lens[b] <= max_context_len
 *   lse          : optional fp32 [B, Hq] natural-log logsumexp (NULL to skip)
 * D in {64, 128}, page_size 64, g <= 16, split_tokens a multiple of 64.
 * Each wavefront streams about split_tokens tokens; a workgroup of 8 covers
 * a chunk of 8 * split_tokens, or up to a quarter more when larger chunks
 * pack the device's workgroups into fewer rounds (never more chunks than
 * the workspace formula counts).  When max_context_len <= 8 * split_tokens
 * this is one kernel and the workspace is not touched.  Otherwise each
 * chunk's workgroup writes its partial and an arrival flag, and the one that
 * sees every flag of its (sequence, KV head) merges the chunks in the same
 * kernel and clears the flags -- when the work list fits one round of the
 * device (spyre_paged_decode_attn_kernels); otherwise a second kernel
 * merges them.  Two calls in flight at once need two workspaces.
 * Empty contexts give zeros (as torch's CPU SDPA does).  Replaces the SDPA
 * overrideable decomposition (torch_spyre/_inductor/decompositions.py:523-609)
 * selected by _fused_sdp_choice (torch_spyre/csrc/attn_utils.cpp:22-37). */
int spyre_paged_decode_attn_f16(const void* q, const void* k_cache, const void* v_cache,
                                const int32_t* block_table, int64_t bt_stride,
                                const int32_t* context_lens, void* out, float* lse,
                                void* workspace, size_t workspace_bytes, int B, int Hq, int Hkv,
                                int D, int page_size, int64_t num_pages, int max_context_len,
                                int split_tokens, float scale, void* stream);

/* Kernels one spyre_paged_decode_attn_f16 call of these sizes launches on
 * the current device: 1 when every context fits one chunk or the chunks
 * merge inside the split kernel (its work list, B * Hkv * chunks items, fits
 * one round of the device's workgroup slots, and the workspace is 16-byte
 * aligned), else 2; negative on bad sizes.  No reference counterpart (a helper for callers that account
 * kernels per step). */
int spyre_paged_decode_attn_kernels(int B, int Hq, int Hkv, int D, int max_context_len, int split_tokens);

/* The two passes of spyre_paged_decode_attn_f16, for callers that schedule
 * them separately (same arguments and workspace; the merge pass reads what
 * the split pass wrote, and no arrival flags are used).  Pass 1 writes
 * every chunk's partial (unnormalised O, running max, row sum) to the
 * workspace; pass 2 combines them into out/lse.
 * No reference counterpart: the reference's SDPA decomposition
 * (torch_spyre/_inductor/decompositions.py:523-609) has no split-KV form. */
int spyre_paged_decode_attn_split_f16(const void* q, const void* k_cache, const void* v_cache,
                                      const int32_t* block_table, int64_t bt_stride,
                                      const int32_t* context_lens, void* workspace,
                                      size_t workspace_bytes, int B, int Hq, int Hkv, int D,
                                      int page_size, int64_t num_pages, int max_context_len,
                                      int split_tokens, float scale, void* stream);
int spyre_paged_decode_attn_merge_f16(const int32_t* context_lens, const void* workspace,
                                      size_t workspace_bytes, void* out, float* lse, int B, int Hq,
                                      int Hkv, int D, int max_context_len, int split_tokens,
                                      void* stream);

/* Host-side check of the addresses the dense decode route (the SDPA entry's
 * one-query calls on dense K / V, below) loads for one 64-token run of a
 * K / V head of which `rows` tokens (1..64) exist, tokens k_row / v_row
 * bytes apart: the largest byte end, from the run's first token, of any K
 * load (k_end) and V load (v_end) that touches memory, and the number of
 * such loads.  Computed from the same address functions as the kernel, on
 * the CPU (no device is used).  The kernel's buffer ranges end at
 * (rows - 1) * row + 2 * D bytes; a result beyond that would read past the
 * view.  No reference counterpart (the reference has no device decode
 * kernel; its decode SDPA is the decomposition of
 * torch_spyre/_inductor/decompositions.py:523-609). */
int spyre_dense_decode_load_extent(int D, int rows, int64_t k_row, int64_t v_row, int64_t* k_end,
                                   int64_t* v_end, int64_t* n_loads);

/* Bytes of the chunk-partial scratch that spyre_paged_decode_attn_noalloc_f16
 * keeps in the library (one copy per GPU, held until the process ends). */
#define SPYRE_DECODE_SCRATCH_BYTES (16u << 20)

/* spyre_paged_decode_attn_f16 without a workspace argument: the chunk
 * partials (and the arrival flags of chunks merged in the split kernel) go
 * to a scratch array the library holds on each GPU, so the call
 * allocates nothing (no hipMalloc / hipFree, no library allocation).
 * Same arguments (less the workspace), kernels and results as
 * spyre_paged_decode_attn_f16.  Returns SPYRE_ENOSPC, before any HIP call,
 * when spyre_paged_decode_attn_workspace_bytes of the call exceeds
 * SPYRE_DECODE_SCRATCH_BYTES (e.g. B 64, 32 / 8 heads, D 128, contexts up
 * to 32768 tokens need 8.1 MiB).  Every call on one GPU shares that GPU's
 * scratch: calls that overlap on one GPU (two streams, two threads) race.
 * No counterpart in the reference: it serves callers that cannot allocate
 * device memory (code under HIP graph capture, serving loops that forbid
 * allocation). */
int spyre_paged_decode_attn_noalloc_f16(const void* q, const void* k_cache, const void* v_cache,
                                        const int32_t* block_table, int64_t bt_stride,
                                        const int32_t* context_lens, void* out, float* lse, int B,
                                        int Hq, int Hkv, int D, int page_size, int64_t num_pages,
                                        int max_context_len, int split_tokens, float scale,
                                        void* stream);

/* Attention mask kinds of spyre_sdpa_fwd_f16. */
#define SPYRE_MASK_NONE 0
#define SPYRE_MASK_F16 1  /* additive fp16 bias                */
#define SPYRE_MASK_F32 2  /* additive fp32 bias                */
#define SPYRE_MASK_BOOL 3 /* uint8/bool: nonzero = attend      */

/* Workspace bytes that cover any spyre_sdpa_fwd_f16 call with an attention
 * mask: V re-laid out with its sticks along tokens, B * Hkv * D *
 * ceil(Skv / 64) * 64 fp16, which the fp32-mask kernel reads.  Calls without
 * a mask (plain or causal) need no workspace. */
size_t spyre_sdpa_fwd_workspace_bytes(int B, int Hkv, int Skv, int D);

/* The workspace one spyre_sdpa_fwd_f16 call needs (same arguments as the
 * call, less the causal flag).  Without a mask: the fp32 partials of a key
 * split, B * Hq * Sq * nsplit * (D + 2) * 4 bytes, when the call's blocks
 * would not fill the device (short query runs, few sequences, long keys),
 * plus, when each KV head's g q heads x Sq queries fit one 32-row tile (the
 * split then merges inside its one kernel), a 4-byte arrival flag per
 * (sequence, KV head, split); the contents need no initialisation.  A
 * call given less (or causal) runs unsplit, same results within the SDPA
 * tolerance, slower.  Decode calls (Sq 1) whose (sequence, KV head, chunk)
 * grid fills at least half the device: when a sequence spans several
 * chunks, their fp32 partials B * Hkv * chunks * g * (D + 2) * 4 bytes and a
 * 4-byte arrival flag per (sequence, KV head, chunk), also without
 * initialisation (the chunks merge in the one kernel).  With a mask: 0 for fp16 / bool masks with
 * key stride 1, a 16-byte aligned pointer, b / h / i strides and Skv of
 * whole 16 bytes (staged in LDS beside K and V as they lie); for other fp16 / bool
 * masks, a copy with 16-byte rows of the mask's non-broadcast extent (then
 * staged the same way); for fp32 masks, spyre_sdpa_fwd_workspace_bytes.  A
 * call whose fp16 / bool mask needs a copy but whose workspace holds only
 * spyre_sdpa_fwd_workspace_bytes runs the fp32-mask kernel instead (same
 * results within the SDPA tolerance, slower).  No reference counterpart:
 * the reference's decomposition (torch_spyre/_inductor/decompositions.py:
 * 523-609) allocates its intermediates itself. */
size_t spyre_sdpa_fwd_call_workspace_bytes(const void* attn_mask, int mask_kind,
                                           const int64_t* mask_strides, int B, int Hq, int Hkv,
                                           int Sq, int Skv, int D);

/* Scaled dot-product attention forward (prefill, any Sq):
 *   out[b,h,i,:] = softmax_j(scale * q[b,h,i,:] . k[b,h/g,j,:] + bias[b,h,i,j]) v[b,h/g,j,:]
 * q [B,Hq,Sq,D], k/v [B,Hkv,Skv,D] fp16 with feature stride 1 and the other
 * strides ({b, h, s}, elements) multiples of 8; 16-byte aligned pointers.
 * bias: none; the mask (kind SPYRE_MASK_*, strides {b, h, i, j} in elements,
 * 0 to broadcast); or, with is_causal, -inf where j > i (top-left aligned).
 * A row with every key masked gives zeros and LSE -inf.
 * out: [B, Sq, Hq, D] contiguous (the layout of the reference's result,
 * returned as its [B,Hq,Sq,D] transpose); lse: optional fp32 [B, Hq, Sq]
 * natural-log logsumexp.  D in {64, 128}; g = Hq / Hkv (GQA).
 * Replaces aten::_scaled_dot_product_fused_attention_overrideable as
 * decomposed by torch_spyre/_inductor/decompositions.py:523-609 (selected by
 * _fused_sdp_choice, torch_spyre/csrc/attn_utils.cpp:22-37), whose logsumexp
 * is left uninitialised (:584-586). */
int spyre_sdpa_fwd_f16(const void* q, const int64_t* q_strides, const void* k,
                       const int64_t* k_strides, const void* v, const int64_t* v_strides,
                       const void* attn_mask, int mask_kind, const int64_t* mask_strides,
                       int is_causal, float scale, void* out, float* lse, void* workspace,
                       size_t workspace_bytes, int B, int Hq, int Hkv, int Sq, int Skv, int D,
                       void* stream);

#ifdef __cplusplus
}
#endif

#endif /* SPYRE_HIP_H */
