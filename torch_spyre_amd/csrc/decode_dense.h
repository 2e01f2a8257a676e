// Dense decode attention (one query per sequence, K / V as dense tensors)
// through the split-KV decode kernels of decode_attn.hip; called by the SDPA
// entry (sdpa_fwd.hip) for the calls it covers.
#pragma once

#include <cstddef>
#include <cstdint>

namespace spyre_hip {

struct DenseDecodePlan {
  bool ok = false;      // the call is covered (sizes only; strides are the caller's check)
  int chunk_pages = 0;  // 64-token runs per chunk (a workgroup's share of a sequence)
  int chunks = 0;       // chunks per sequence
  size_t ws_bytes = 0;  // chunks > 1: fp32 chunk partials and a flag per chunk, else 0
  int waves = 8;        // wavefronts per item (= per workgroup): 8, or 4 (twice the runs each)
  bool fused = false;   // chunks > 1 merged inside the kernel (else the merge pass)
};

// The plan for q [B, Hq, 1, D] against K / V of Skv tokens: covered when
// D in {64, 128}, Hq / Hkv <= 16 and the (sequence, KV head, chunk) grid fills at
// least half of the device's workgroup slots (chunks of 8 wavefronts x
// 64-512 tokens).
DenseDecodePlan dense_decode_plan(int B, int Hq, int Hkv, int Skv, int D);

// A nonzero value, new on every call (process-wide): the arrival-flag value
// of a kernel whose workgroups merge their partials in the same launch.
uint32_t next_call_ticket();

// Launches the plan: q strides {b, h} and K / V strides {b, h, s} in
// elements (feature stride 1, 16-byte aligned rows, token strides below
// 2^23); out [B, Hq, D] contiguous fp16; lse optional [B, Hq] fp32; the
// workspace (16-byte aligned) holds plan.ws_bytes and needs no
// initialisation: the flags a call sets are cleared by the same call.
int dense_decode_launch(const DenseDecodePlan& plan, const void* q, const int64_t* q_strides, const void* k,
                        const int64_t* k_strides, const void* v, const int64_t* v_strides, void* out, float* lse,
                        void* workspace, int B, int Hq, int Hkv, int Skv, int D, float scale, void* stream);

}  // namespace spyre_hip
