// Persistent MoE decode megakernel for MI355X (gfx950, CDNA4).
//
// One workgroup per compute unit runs its instruction queue in order
// (instruction layout: megakernels/instructions.py:97-119).  Workers meet only
// through int32 counters in HBM.  Data that one workgroup produces and
// another consumes within a launch (SiLU rows, hidden rows, router outputs)
// is written with agent-scope (device-coherent, write-through) stores and
// read with agent-scope loads; an arrival is all waves' stores completed
// (s_waitcnt) followed by a relaxed agent-scope fetch-add, and a wait is a
// bounded spin of relaxed agent-scope loads.  No L2 write-back or invalidate
// is issued: on MI355X those serialise per XCD and cost ~15 us each when all
// compute units issue them together, while the coherent accesses cost well
// under a microsecond.  There is no loader/consumer/storer split as
// in the reference's warp-specialised VM (include/megakernel.cuh:118-140):
// every wave issues its own 16-byte weight loads and does its own math.
//
// Hot-path opcodes (demos/mixtral/*.cu in the reference):
//   5 RmsRouterUpgate       RMSNorm + router + top-2 + gate/up GEMV + SiLU
//   6 ExpertDownProjFused   down GEMV of both experts + weighted residual add
//   8 SpeculativeExpertPredict  top-2 prediction from the pre-attention residual
//
// Numerics follow megakernels/mixtral/python_vm.py (bf16 storage, fp32
// accumulation) with its bf16 rounding points:
//   normed   = bf16(w_ln * bf16(x * 1/sqrt(mean(x^2) + eps)))
//   logits   = W_r . normed (fp32) [+ bias]
//   scores   = bf16(p_i / (p_0 + p_1)), p = softmax(logits), top-2 by p
//   silu_out = bf16(bf16(silu(bf16(g))) * bf16(u))
//   h        = bf16(h + bf16(s_j * bf16(d_j)))   for j = 0, 1 in order
//
// GEMV mapping (batch-1 matvec is HBM-bound, ~1 flop/byte, so no MFMA): a
// wave owns whole output rows.  Lane l of a wave covers columns
// [512c + 8l, 512c + 8l + 8) of chunk c, so one wave-wide dwordx4 load reads
// 1 KiB of contiguous weights.  Weights go HBM -> VGPR with non-temporal
// loads; the activation vector is staged once per instruction in LDS; each
// bf16 pair is widened exactly to fp32 and fused-multiply-added into an fp32
// accumulator; the row sum is a 64-lane DPP reduction.

#include <hip/hip_runtime.h>

#include <math.h>
#include <algorithm>
#include <cctype>
#include <cerrno>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <mutex>
#include <stddef.h>
#include <stdint.h>

#include "mk_llama.h"
#include "mk_mixtral.h"

#ifndef MK_THREADS
#define MK_THREADS 512
#endif
#ifndef MK_NT_LOADS
#define MK_NT_LOADS 1
#endif
// Work sharing (opcode 5): the last MK_TAIL_ITEMS items of every opcode-5
// instruction are claimed through a cursor in HBM, so the other workers of
// its group (MK_POOL_GROUP consecutive workers, which sit on different XCDs)
// can take them once their own instruction is done.
#ifndef MK_TAIL_ITEMS
#define MK_TAIL_ITEMS 16
#endif
#ifndef MK_POOL_GROUP
#define MK_POOL_GROUP 8
#endif
// O-projection rows staged in LDS by a preceding reduction (stage_oproj_rows).
#ifndef MK_OSTAGE
#define MK_OSTAGE 1
#endif
// Spin back-off: a waiting workgroup polls its counter every ~64 * N clocks,
// N doubling from 1 to MK_SPIN_SLEEP_MAX (a launch field), so hundreds of
// idle workgroups do not keep the memory channels busy while others still
// stream weights.  Same-process A/B of the cap: 16 beats 4 by 0.4 % at
// config 3 and 0.2 % at configs 4 and 5; 32 is level with 16, 64 slower.
#ifndef MK_SPIN_SLEEP_MAX
#define MK_SPIN_SLEEP_MAX 16
#endif
#ifndef MK_CLAIM_LOOKAHEAD
#define MK_CLAIM_LOOKAHEAD 1
#endif
// Opcode 6: each wave loads its two first items (both register sets)
// before the wait for opcode 5 (0 = after it).
#ifndef MK_EARLY_LOADS
#define MK_EARLY_LOADS 1
#endif
// Opcode-6 cache warming while waiting for opcode 5: items per wave (0 = off).
#ifndef MK_PF_ROUNDS
#define MK_PF_ROUNDS 1
#endif

// Dense VM: at most this many opcode-5 items (gate and up rows) staged in LDS
// by the preceding opcode 4 (fewer when the LDS left over holds fewer).
#ifndef MK_STAGE_ITEMS
#define MK_STAGE_ITEMS 16
#endif
// Machine-code bytes of each kernel, read into L2 as the kernel runs
// (code_prefetch).  The build measures them from the compiler's output of
// the same source and compiles the library a second time with them; only
// host code uses them, so the device code of both compiles is identical.
// 0: no prefetch (a library compiled in one pass).
#ifndef MK_CODE_LEN_LLAMA
#define MK_CODE_LEN_LLAMA 0
#endif
#ifndef MK_CODE_LEN_E8_ATTN
#define MK_CODE_LEN_E8_ATTN 0
#endif
#ifndef MK_CODE_LEN_E0_ATTN
#define MK_CODE_LEN_E0_ATTN 0
#endif
#ifndef MK_CODE_LEN_E8
#define MK_CODE_LEN_E8 0
#endif
#ifndef MK_CODE_LEN_E0
#define MK_CODE_LEN_E0 0
#endif

namespace {

constexpr int kThreads = MK_THREADS;
constexpr int kWaves = kThreads / 64;
constexpr int kChunkElems = 512;  // bf16 columns covered by one wave-wide 16 B/lane load
// More than half of the 160 KiB LDS: the dispatcher can then place only one
// workgroup per compute unit, so a grid of #CU workers covers every CU once.
constexpr int kMinLdsBytes = 84 * 1024;
constexpr uint32_t kTicksPerUs = 100;  // s_memrealtime runs at 100 MHz
constexpr int kCachePolicySc1 = 16;     // buffer-load cache policy: device scope
// Work-sharing scratch (int32): [0] exit counter, then a (cursor, done) pair
// per instruction slot w * queue_len + q.
constexpr int kScratchSlotBase = 16;
// Spread layer counters: arrivals on the counter at index 0 of a (layer,
// opcode) row of the barrier tensor go to one of kSpread counters in
// library scratch instead (the arriving workgroup's XCD picks it, blocks
// spreading over XCDs round-robin), kSpreadAlign ints apart; waiters add the
// row-0 counter and its kSpread parts, and the last workgroup of the launch
// folds the parts back into the barrier tensor.
constexpr int kSpread = 8;
constexpr int kXcds = 8;  // MI355X: workgroup w runs on XCD w % 8 (round-robin dispatch)
constexpr int kSpreadAlign = 1024;
// opcodes whose layer counters are spread, per kernel (bit k = opcode k),
// from same-process A/B runs (MK_SPREAD overrides them): none spread costs
// config 3 5.4 % and config 4 1.2 %; adding opcode 3's counter (the
// reductions' arrivals, polled by every O projection) gains config 3 0.5 %
// and config 4 0.2 %; opcodes 7 and 8 change nothing
constexpr int32_t kSpreadDenseOps = (1 << 3) | (1 << 4) | (1 << 5) | (1 << 6);
constexpr int32_t kSpreadMixtralOps = (1 << 3) | (1 << 4) | (1 << 5) | (1 << 6);
constexpr int32_t kSpreadMoeOps = 0;
constexpr int kPoolGroup = MK_POOL_GROUP;
constexpr int kMaxPoolIns = 64;  // opcode-5 instructions per (layer, group) that can be shared
constexpr int kPoolWindow = 8;  // queue slots per group member pool_scan_near looks at
static_assert(kMaxPoolIns <= 64, "one lane per group instruction");
constexpr int kRowBatchLds = 64;  // rows per opcode-6 batch (partial sums in LDS)
constexpr int kMaxSegments = 10;  // column segments per opcode-6 row (F <= 10 * 7 * 512)
constexpr int kMaxIntermediate = 32768;  // largest intermediate size the launch accepts
constexpr int kMaxMerge = 8;      // consecutive opcode-5 instructions of a layer run as one item pool
#ifndef MK_GROUP_CHUNKS
#define MK_GROUP_CHUNKS 7
#endif
#ifndef MK_ITEM_ROWS
#define MK_ITEM_ROWS 1
#endif
constexpr int kGroupChunks = MK_GROUP_CHUNKS;  // overlapped opcode 6: 512-column chunks per column group
constexpr int kItemRows = MK_ITEM_ROWS;        // overlapped opcode 6: rows per item (both experts)
constexpr int kMaxGroups = 8;     // overlapped opcode 6: column groups per row (F <= 8 * 4 * 512)
static_assert(kRowBatchLds * 2 * kMaxSegments >= 32 * 2 * kMaxGroups, "overlapped opcode-6 partials fit in sh.part");

static_assert(kThreads % 64 == 0 && kThreads <= 1024, "wave64 workgroup");

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
// Instruction words are read through the constant address space: the kernel
// never writes them, so uniform reads become scalar loads, which wait on
// their own counter instead of queueing behind the wave's outstanding
// weight loads (a vector load of an instruction word waits for all of them).
typedef const __attribute__((address_space(4))) int32_t ins_t;
typedef __attribute__((address_space(3))) void lds_void_t;          // LDS pointer (global_load_lds destination)
typedef const __attribute__((address_space(1))) void global_void_t;  // global pointer (global_load_lds source)

// Parameters of the attention opcodes (1-4) and the LM head (7).  They sit
// in the kernel's argument block (KParams::attn_params), one copy per
// launch, and are read through the constant address space like the
// instruction words: the kernel never writes them, so the reads are scalar
// loads (cached, and not queued behind the wave's outstanding weight loads
// as vector loads would be), and the opcode-5/6 loops keep none of them in
// registers.
struct AttnParams {
    const uint16_t *qkv, *attn_ln, *oproj, *lm_norm, *lm_head;
    uint16_t *kc, *vc, *q_rope, *attn_out, *logits;
    const float *rope_cos, *rope_sin;
    float *lse_int, *out_int;
    int32_t Hq, Hkv, D, V, T, P;
    int32_t qkv_bs, kv_bs, lm_bs, lm_red;
    float attn_scale;
    int32_t skip_red;
    int32_t kv_ring;  // opcode-2 LDS ring chunks (kAttnSub or kKvRingMax)
};

struct KParams {
    const int32_t *instructions;
    int32_t *timings;
    int32_t *bar;
    int32_t *status;
    const uint16_t *gate;
    const uint16_t *up;
    const uint16_t *down;
    const uint16_t *router;
    const uint16_t *predictor;
    const uint16_t *ffn_ln;
    const float *router_bias;
    uint16_t *hidden;
    uint16_t *silu;
    uint16_t *normed_out;
    int32_t *sel_idx;
    uint16_t *sel_score;
    int32_t *pred_idx;
    int32_t queue_len;
    int32_t num_layers, H, F, E;
    int32_t bar_ops, bar_width;
    int32_t expert_bs, down_bs, oproj_bs;
    float eps;
    uint32_t timeout_ticks;
    int32_t *scratch;
    int32_t work_sharing;
    int32_t spin_max;  // longest back-off between polls, in s_sleep(1) units
    int32_t tail_items;    // opcode-5 work sharing: items per instruction claimed through its cursor
    int32_t early_loads;   // opcode 6: each wave's two first items loaded before the wait (0/1)
    int32_t pf_rounds;     // opcode 6: cache-warming rounds while opcode 5 still runs elsewhere
    // opcode 3 streams its worker's next O-projection rows into LDS while it
    // waits (stage_oproj_rows): on for the Mixtral VM, off for the dense one
    int32_t ostage;
    // attention side and LM head (opcodes 1-4, 7): attn == 0 when absent
    int32_t attn;
    uint32_t pos;  // pos_id: changes every decode step, so it stays a kernel argument
    // arrivals on [l][5][0] that complete a layer's down-projection (Mixtral:
    // 2 * H / down_bs; dense Llama: (F / red_cols) * (H / down_bs))
    int32_t down_arrivals;
    int32_t red_cols;  // dense down-projection column chunk (matvec_reduction_size)
    // decode-driver extension (NULL: off): the last workgroup to exit writes
    // argmax(logits) to argmax_out and, with next_embed, copies that row of
    // the embedding table into hidden (the next step's input)
    int64_t *argmax_out;
    const uint16_t *next_embed;
    // with argmax_out: the last workgroup also zeroes the barrier tensor (1)
    // and the logits (2) for the next launch
    int32_t reset_next;
    // opcode-5 items (gate and up rows) staged in LDS while a workgroup waits
    // anyway -- dense VM: by opcode 4 or 5; Mixtral whole-model launches: by
    // opcode 5, from opcode 8's prediction -- and where (u32x4 index into the
    // dynamic LDS); 0: off
    int32_t stage_items;
    int32_t stage_off16;
    // nonzero: every instruction waits for its inputs before it issues any
    // load, and nothing is staged for a later instruction (the prefetch-off
    // side of an A/B; stage_items is then 0).  Whole-model and dense
    // launches; the MoE-only kernel ignores it.
    int32_t late_loads;
    int32_t lds_bytes;  // dynamic LDS of the launch
    // opcode-5/6 overlap (NULL: off): finished SiLU rows of both selected
    // experts per (layer, 512-row column chunk of F), counted by opcode 5 as
    // its instructions complete; opcode 6 then starts on the column groups
    // that are complete instead of waiting for the whole layer
    int32_t *chunk_ctr;
    int32_t scratch_clear;  // scratch ints from kScratchSlotBase the last workgroup zeroes
    // dense VM with argmax_out: per workgroup (value, index) of the best
    // logit its LM-head instructions wrote (2 ints each), which the exit
    // argmax reduces instead of reading every logit; null: read the logits
    int32_t *lm_cand;
    // spread layer counters (NULL: off): kSpread parts of spread_rows
    // (layer, opcode) rows, spread_stride ints apart
    int32_t *spread;
    int32_t spread_rows, spread_stride;
    int32_t spread_ops;  // bit k: rows of opcode k are spread
    // exact division by bar_width and bar_ops for barrier offsets below
    // bar_ints (< 2^16 whenever spread is set): q = umulhi(n, ceil(2^32 / d))
    uint32_t bar_width_magic, bar_ops_magic;
    int32_t bar_ints;
    // bytes of the launched kernel's machine code that code_prefetch reads
    // into L2 (at most the kernel's length; 0: off)
    uint32_t code_len;
    AttnParams attn_params;  // read only through attn_of()
};

// The launch parameters, read in place from the kernel-argument segment
// (KParams is the kernel's only argument, at offset 0): scalar loads where a
// field is used, instead of every field held in registers for the whole
// persistent loop.
typedef const __attribute__((address_space(4))) KParams kp_c;
__device__ __forceinline__ kp_c &kparams() {
    const __attribute__((address_space(4))) char *kernarg =
        (const __attribute__((address_space(4))) char *)__builtin_amdgcn_kernarg_segment_ptr();
    return *reinterpret_cast<kp_c *>(kernarg);
}

// The launch's attention parameters, addressed in the kernel-argument
// segment itself (KParams is the kernel's only argument, at offset 0).
typedef const __attribute__((address_space(4))) AttnParams attn_c;
__device__ __forceinline__ attn_c &attn_of(kp_c &) {
    const __attribute__((address_space(4))) char *kernarg =
        (const __attribute__((address_space(4))) char *)__builtin_amdgcn_kernarg_segment_ptr();
    return *reinterpret_cast<attn_c *>(kernarg + offsetof(KParams, attn_params));
}

// Per-workgroup state that outlives a single instruction.
struct SharedState {
    float red[kWaves * MK_MAX_EXPERTS];
    float red_ss[kWaves];
    float bias[MK_MAX_EXPERTS];
    int route_layer;  // layer whose routing below was computed here, -1 none
    int route_idx[2];
    float route_score[2];  // bf16 score values widened to fp32
    int flag;
    uint32_t touch[64];  // landing words of the next-instruction touch and the code prefetch (never read)
    float lm_v;  // the best logit this workgroup's dense LM-head rows produced (lm_idx -1: none)
    int lm_idx;
    int next_item;  // per-instruction item counter shared by the waves
    float part[kRowBatchLds * 2 * kMaxSegments];  // opcode-6 partial sums: [row][slot][segment]
    // opcode-5 instructions of this worker's group for the current layer, in
    // (worker, slot) order: instruction slot, first FFN row, rows
    int pool_n;
    int wave_cnt[kWaves];
    int pool_slot[kMaxPoolIns], pool_row0[kMaxPoolIns], pool_nrows[kMaxPoolIns];
    int spec_e[2];  // opcode 5: experts opcode 8 predicted for the layer (-1: none yet)
    // dense VM: queue slot whose first stage_n opcode-5 items opcode 4 staged
    // in LDS (-1: none)
    int stage_slot, stage_n;
    // queue slot of the opcode 4 whose weight rows opcode 3 staged in LDS
    // (-1: none)
    int ostage_slot;
    // opcode 5 over consecutive instructions of one layer (kMaxMerge at
    // most): first FFN row, rows, first pooled item, finished items
    int grp_row0[kMaxMerge], grp_nrows[kMaxMerge], grp_first[kMaxMerge + 1], grp_done[kMaxMerge];
    int ready_mask;  // opcode 6: column groups whose SiLU rows are complete
};

struct Ctx {
    int worker;
    int slot;
};

// ---------------------------------------------------------------------------
// scalar helpers
// ---------------------------------------------------------------------------

__device__ __forceinline__ float bf2f(uint32_t h) { return __uint_as_float(h << 16); }

// fp32 -> bf16 bits, round to nearest even; NaN -> canonical quiet NaN.
__device__ __forceinline__ uint32_t f2bf(float f) {
    const uint32_t u = __float_as_uint(f);
    if ((u & 0x7fffffffu) > 0x7f800000u) return 0x7fc0u;
    return (u + 0x7fffu + ((u >> 16) & 1u)) >> 16;
}

__device__ __forceinline__ float rbf(float f) { return bf2f(f2bf(f)); }

// Device-coherent accesses for data shared between workgroups of a launch.
__device__ __forceinline__ void st_dev16(uint16_t *p, uint32_t v) {
    __hip_atomic_store(p, (uint16_t)v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_dev32(void *p, uint32_t v) {
    __hip_atomic_store(reinterpret_cast<uint32_t *>(p), v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint32_t ld_dev16(const uint16_t *p) {
    return __hip_atomic_load(const_cast<uint16_t *>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint32_t ld_dev32(const void *p) {
    return __hip_atomic_load(const_cast<uint32_t *>(reinterpret_cast<const uint32_t *>(p)), __ATOMIC_RELAXED,
                             __HIP_MEMORY_SCOPE_AGENT);
}
// 16-byte device-coherent load of base + byte_off (base uniform across the
// wave): a raw buffer load with the sc1 cache policy.
__device__ __forceinline__ u32x4 ld_dev128(const void *base, uint32_t byte_off) {
    const __amdgpu_buffer_rsrc_t r =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), (short)0, 0x7fffffff, 0x00020000);
    return __builtin_amdgcn_raw_buffer_load_b128(r, byte_off, 0, kCachePolicySc1);
}
// 4-byte device-coherent load of base + byte_off (base uniform across the
// wave) as a raw buffer load with the sc1 policy: unlike an atomic load,
// the compiler may issue many of them back to back.
__device__ __forceinline__ uint32_t ld_dev32_at(const void *base, uint32_t byte_off) {
    const __amdgpu_buffer_rsrc_t r =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), (short)0, 0x7fffffff, 0x00020000);
    return __builtin_amdgcn_raw_buffer_load_b32(r, byte_off, 0, kCachePolicySc1);
}
__device__ __forceinline__ void st_dev128(u32x4 *p, u32x4 v) {
    uint32_t *q = reinterpret_cast<uint32_t *>(p);
    st_dev32(q, v.x);
    st_dev32(q + 1, v.y);
    st_dev32(q + 2, v.z);
    st_dev32(q + 3, v.w);
}

__device__ __forceinline__ u32x4 load_stream(const u32x4 *p) {
#if MK_NT_LOADS
    return __builtin_nontemporal_load(p);
#else
    return *p;
#endif
}

// 8-element bf16 dot product accumulated in fp32: each bf16 is widened
// exactly (low half << 16, high half & 0xffff0000) and multiplied-added with
// fmaf.
__device__ __forceinline__ float dot2_fma(uint32_t w, uint32_t a, float acc) {
    acc = fmaf(__uint_as_float(w << 16), __uint_as_float(a << 16), acc);
    return fmaf(__uint_as_float(w & 0xffff0000u), __uint_as_float(a & 0xffff0000u), acc);
}

__device__ __forceinline__ float dot8(u32x4 w, u32x4 a, float acc) {
    acc = dot2_fma(w.x, a.x, acc);
    acc = dot2_fma(w.y, a.y, acc);
    acc = dot2_fma(w.z, a.z, acc);
    acc = dot2_fma(w.w, a.w, acc);
    return acc;
}

template <int CTRL, int ROW_MASK = 0xf>
__device__ __forceinline__ float dpp_add_src(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, ROW_MASK, 0xf, false));
}

// Sum over the 64 lanes with DPP: pairs within quads, quads, half rows,
// rows (16 lanes), then row 0 -> 1 and 2 -> 3 (row_bcast15) and rows 0-1 ->
// 2-3 (row_bcast31); lane 63 holds the total, which is returned to every
// lane.  Fixed order, so the result is deterministic.
__device__ __forceinline__ float wave_sum(float v) {
    v += dpp_add_src<0xb1>(v);        // quad_perm [1, 0, 3, 2]
    v += dpp_add_src<0x4e>(v);        // quad_perm [2, 3, 0, 1]
    v += dpp_add_src<0x141>(v);       // row_half_mirror
    v += dpp_add_src<0x140>(v);       // row_mirror
    v += dpp_add_src<0x142, 0xa>(v);  // row_bcast15 into rows 1 and 3
    v += dpp_add_src<0x143, 0xc>(v);  // row_bcast31 into rows 2 and 3
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
}

// Workgroup sum.  `red` must not be reused before the next workgroup
// barrier.
__device__ __forceinline__ float block_sum(float v, float *red) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    v = wave_sum(v);
    if (lane == 0) red[wave] = v;
    __syncthreads();
    float s = 0.f;
#pragma unroll
    for (int i = 0; i < kWaves; ++i) s += red[i];
    return s;
}

__device__ __forceinline__ float sumsq2(uint32_t x) {
    const float a = bf2f(x & 0xffffu), b = bf2f(x >> 16);
    return a * a + b * b;
}

// python_vm rms_norm on two packed bf16 values: bf16(w * bf16(x * r)).
__device__ __forceinline__ uint32_t norm2(uint32_t x, uint32_t w, float r) {
    const float n0 = rbf(bf2f(x & 0xffffu) * r), n1 = rbf(bf2f(x >> 16) * r);
    return f2bf(bf2f(w & 0xffffu) * n0) | (f2bf(bf2f(w >> 16) * n1) << 16);
}

// ---------------------------------------------------------------------------
// timing, status, barriers
// ---------------------------------------------------------------------------

__device__ __forceinline__ void stamp(int32_t *t, int slot) {
    if (t != nullptr && threadIdx.x == 0) t[slot] = (int32_t)(uint32_t)__builtin_amdgcn_s_memrealtime();
}

// The next instruction's two 64-byte lines, read once into L2 by lanes 0
// and 1 of the last wave (a 4-byte global_load_lds writes the word of lane
// i at the LDS base + 4 i: sh.touch[0..1], never read): the scalar loads
// that fetch it when its turn comes then find it there instead of in
// memory.
__device__ __forceinline__ void touch_next_instruction(kp_c &p, SharedState &sh, ins_t *ins, int q) {
    const int t = (int)threadIdx.x - (kThreads - 64);
    if (q + 1 < p.queue_len && t >= 0 && t < 2) {
        const uintptr_t a = reinterpret_cast<uintptr_t>(ins + MK_INTS_PER_INSTRUCTION) + (uintptr_t)t * 64u;
        __builtin_amdgcn_global_load_lds((global_void_t *)a, (lds_void_t *)sh.touch, 4, 0, 0);
    }
}

// First byte of the running kernel's machine code.  Kernels start on
// 256-byte boundaries and every kernel calls this first thing, within its
// first 256 bytes (the build checks that in the compiler's output), so the
// program counter rounded down to 256 bytes is the entry.
__device__ __forceinline__ uint64_t kernel_code_base() {
    uint64_t pc;
    asm volatile("s_getpc_b64 %0" : "=s"(pc));
    return pc & ~(uint64_t)255;
}

// The kernel's machine code, kept in L2: at the start of every instruction
// the last-but-one wave reads 4 bytes of each 128-byte line of one 32nd of
// the code (global_load_lds into sh.touch, never read), workgroup w slice
// (w / 8 + q) mod 32, so the 32 workgroups of an XCD (blockIdx mod 8) cover
// all of it at every round of instruction starts.  The weight stream evicts
// the code from L2 within a layer; without this, a stage's first
// instructions wait ~0.9 us for each instruction-cache line from HBM (about
// 185,000 instruction-cache misses per config-4 step), on the critical path
// of whichever workgroup finished the previous stage last.  Reads stay
// below code + p.code_len, at most the kernel's length.
// The 32 KiB of machine code that follow the program counter where this is
// called (the handler about to run), read into L2 in one batch by the
// third-last wave: the instruction cache's misses as the handler starts then
// find their lines in L2 instead of fetching them from HBM one after
// another.  Same-process A/B against code_prefetch alone: config 4 +0.3 to
// +0.4 %, config 3 +0.2 %; 64 KiB measured 1 % slower at config 3.  Reads
// stay inside [code, code + p.code_len).
__device__ __forceinline__ void handler_prefetch(kp_c &p, SharedState &sh, uint64_t code) {
    const int t = (int)threadIdx.x - (kThreads - 192);
    if (p.code_len == 0 || t < 0 || t >= 64) return;
    uint64_t pc;
    asm volatile("s_getpc_b64 %0" : "=s"(pc));
    const uint64_t end = code + (p.code_len & ~127u), base = pc & ~(uint64_t)127;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const uint64_t a = base + ((uint64_t)(t + 64 * k) << 7);
        if (a < end) __builtin_amdgcn_global_load_lds((global_void_t *)a, (lds_void_t *)sh.touch, 4, 0, 0);
    }
}

__device__ __forceinline__ void code_prefetch(kp_c &p, SharedState &sh, uint64_t code, int q) {
    const int t = (int)threadIdx.x - (kThreads - 128);
    const uint32_t lines = p.code_len >> 7;
    if (lines == 0 || t < 0 || t >= 64) return;
    const uint32_t per = (lines + 31) >> 5, j = ((uint32_t)(blockIdx.x >> 3) + (uint32_t)q) & 31u;
    const uint32_t end = min(j * per + per, lines);
    for (uint32_t l = j * per + (uint32_t)t; l < end; l += 64u)
        __builtin_amdgcn_global_load_lds((global_void_t *)(code + ((uint64_t)l << 7)), (lds_void_t *)sh.touch, 4, 0,
                                         0);
}

__device__ __forceinline__ int32_t *bar_at(kp_c &p, int layer, int opcode) {
    return p.bar + ((size_t)layer * p.bar_ops + (opcode - 1)) * p.bar_width;
}

__device__ __forceinline__ bool aborted(kp_c &p) {
    return __hip_atomic_load(p.status, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != 0;
}

// Record the first failure; called by one lane.
__device__ __forceinline__ void report_error_lane(kp_c &p, int code, const Ctx &c, int opcode, int layer, int expected,
                                  int seen) {
    int zero = 0;
    if (__hip_atomic_compare_exchange_strong(p.status, &zero, code, __ATOMIC_RELAXED, __ATOMIC_RELAXED,
                                             __HIP_MEMORY_SCOPE_AGENT)) {
        p.status[MK_STATUS_WORKER] = c.worker;
        p.status[MK_STATUS_SLOT] = c.slot;
        p.status[MK_STATUS_OPCODE] = opcode;
        p.status[MK_STATUS_LAYER] = layer;
        p.status[MK_STATUS_EXPECTED] = expected;
        p.status[MK_STATUS_SEEN] = seen;
    }
}

// Record the first failure (thread 0 of the reporting workgroup only).
__device__ __forceinline__ void report_error(kp_c &p, int code, const Ctx &c, int opcode, int layer, int expected, int seen) {
    if (threadIdx.x == 0) report_error_lane(p, code, c, opcode, layer, expected, seen);
}

// Row of the spread counter table for `ctr` (the counter at index 0 of a
// (layer, opcode) row of the barrier tensor), or -1 (not spread).
// Divisions by the barrier tensor's row lengths are multiplications by
// host-computed reciprocals (exact for n, d < 2^16: the error n (m d - 2^32)
// / (d 2^32) stays below 1 / d), a few scalar instructions where a 64-bit
// division would take some 150 at every arrival and wait.
__device__ __forceinline__ int spread_row(kp_c &p, const int32_t *ctr) {
    if (p.spread == nullptr) return -1;
    const long d = ctr - p.bar;
    if (d < 0 || d >= p.bar_ints) return -1;
    const uint32_t off = (uint32_t)d;
    const uint32_t row = __umulhi(off, p.bar_width_magic);
    if (row * (uint32_t)p.bar_width != off || (int)row >= p.spread_rows) return -1;
    const uint32_t op0 = row - __umulhi(row, p.bar_ops_magic) * (uint32_t)p.bar_ops;
    if (!((p.spread_ops >> (op0 + 1)) & 1)) return -1;
    return (int)row;
}

// One lane adds n arrivals to counter `ctr`.  A few hundred workgroups that
// finish a stage together all add to one address, and the memory channel
// applies those atomics one at a time (~15 ns each): the last of 256
// O-projection arrivals landed ~4 us after the stage ended.  A spread
// counter's arrivals go to this XCD's part instead, 32 per part.
__device__ __forceinline__ void arrive_add(kp_c &p, int32_t *ctr, int n) {
    const int row = spread_row(p, ctr);
    int32_t *dst = row < 0 ? ctr : p.spread + (size_t)(blockIdx.x % kSpread) * p.spread_stride + row;
    __hip_atomic_fetch_add(dst, n, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ void arrive(kp_c &p, int32_t *ctr, int n) {
    if (threadIdx.x == 0) arrive_add(p, ctr, n);
}

// Current value of counter `ctr` (row `row` of the spread table, or -1),
// read by one lane: the counter and its kSpread parts, all loads in flight
// together.
__device__ __forceinline__ int counter_value(kp_c &p, const int32_t *ctr, int row) {
    int v = (int)ld_dev32(ctr);
    if (row >= 0) {
        uint32_t part[kSpread];
#pragma unroll
        for (int k = 0; k < kSpread; ++k) part[k] = ld_dev32(p.spread + (size_t)k * p.spread_stride + row);
#pragma unroll
        for (int k = 0; k < kSpread; ++k) v += (int)part[k];
    }
    return v;
}

// Whether counter `ctr` has reached `expected`, for the workgroup (thread 0
// reads it; ends with a workgroup barrier).
__device__ __forceinline__ bool counter_reached(kp_c &p, SharedState &sh, const int32_t *ctr, int expected) {
    if (threadIdx.x == 0) sh.flag = counter_value(p, ctr, spread_row(p, ctr)) >= expected;
    __syncthreads();
    const bool r = sh.flag != 0;
    __syncthreads();
    return r;
}

// Wait until counter `ctr` >= expected.  Thread 0 spins; the result is
// broadcast.  Returns false (uniformly) on time-out or when another worker
// has failed.
__device__ __forceinline__ bool wait_ge(kp_c &p, SharedState &sh, int32_t *ctr, int expected, const Ctx &c, int opcode,
                        int layer) {
    if (threadIdx.x == 0) {
        const int row = spread_row(p, ctr);
        int ok = 1;
        int v = counter_value(p, ctr, row);
        if (v < expected) {
            const uint64_t t0 = __builtin_amdgcn_s_memrealtime();
            int nap = 1;
            for (;;) {
                for (int i = 0; i < nap; ++i) __builtin_amdgcn_s_sleep(1);
                if (nap < p.spin_max) nap *= 2;
                v = counter_value(p, ctr, row);
                if (v >= expected) break;
                if (aborted(p)) {
                    ok = 0;
                    break;
                }
                if (__builtin_amdgcn_s_memrealtime() - t0 > (uint64_t)p.timeout_ticks) {
                    report_error(p, MK_ERR_TIMEOUT, c, opcode, layer, expected, v);
                    ok = 0;
                    break;
                }
            }
        }
        sh.flag = ok;
    }
    __syncthreads();
    const bool ok = sh.flag != 0;
    __syncthreads();
    return ok;
}

// Make every wave's global stores complete, then join the workgroup (a
// workgroup barrier alone does not wait for other waves' outstanding stores).
__device__ __forceinline__ void drain_and_sync() {
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
}

// ---------------------------------------------------------------------------
// GEMV core: two rows at once, N chunks of 512 columns each
// ---------------------------------------------------------------------------

template <int N>
__device__ __forceinline__ void dot_pair_n(const u32x4 *__restrict__ wa, const u32x4 *__restrict__ wb,
                                           const u32x4 *xa, const u32x4 *xb, float &acc_a, float &acc_b) {
    u32x4 ra[N], rb[N];
#pragma unroll
    for (int i = 0; i < N; ++i) {
        ra[i] = load_stream(wa + i * 64);
        rb[i] = load_stream(wb + i * 64);
    }
#pragma unroll
    for (int i = 0; i < N; ++i) {
        acc_a = dot8(ra[i], xa[i * 64], acc_a);
        acc_b = dot8(rb[i], xb[i * 64], acc_b);
    }
}

// Per-lane partial dot products of rows a and b (each nc * 512 bf16) with
// LDS activations xa and xb.  Caller reduces across the wave.
__device__ __forceinline__ void dot_pair(const uint16_t *row_a, const uint16_t *row_b, const u32x4 *xa,
                                         const u32x4 *xb, int nc, int lane, float &acc_a, float &acc_b) {
    const u32x4 *wa = reinterpret_cast<const u32x4 *>(row_a) + lane;
    const u32x4 *wb = reinterpret_cast<const u32x4 *>(row_b) + lane;
    xa += lane;
    xb += lane;
    int c = 0;
    for (; c + 8 <= nc; c += 8) dot_pair_n<8>(wa + c * 64, wb + c * 64, xa + c * 64, xb + c * 64, acc_a, acc_b);
    switch (nc - c) {
    case 7: dot_pair_n<7>(wa + c * 64, wb + c * 64, xa + c * 64, xb + c * 64, acc_a, acc_b); break;
    case 6: dot_pair_n<6>(wa + c * 64, wb + c * 64, xa + c * 64, xb + c * 64, acc_a, acc_b); break;
    case 5: dot_pair_n<5>(wa + c * 64, wb + c * 64, xa + c * 64, xb + c * 64, acc_a, acc_b); break;
    case 4: dot_pair_n<4>(wa + c * 64, wb + c * 64, xa + c * 64, xb + c * 64, acc_a, acc_b); break;
    case 3: dot_pair_n<3>(wa + c * 64, wb + c * 64, xa + c * 64, xb + c * 64, acc_a, acc_b); break;
    case 2: dot_pair_n<2>(wa + c * 64, wb + c * 64, xa + c * 64, xb + c * 64, acc_a, acc_b); break;
    case 1: dot_pair_n<1>(wa + c * 64, wb + c * 64, xa + c * 64, xb + c * 64, acc_a, acc_b); break;
    default: break;
    }
}

// The first item of a wave in matvec_rows (rows r0 + 2 * wave and the next),
// first min(nc, 8) chunks, loaded ahead: issued before a wait on inputs that
// the weights do not depend on, so the weight stream overlaps the wait.
constexpr int kAheadChunks = 8;
struct PairAhead {
    u32x4 a[kAheadChunks], b[kAheadChunks];
};

__device__ __forceinline__ void pair_ahead_load(PairAhead &r, const uint16_t *mat, size_t ld, int col0, int nc,
                                                int r0, int nrows) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    if (2 * wave >= nrows) return;
    const int ra = r0 + 2 * wave;
    const u32x4 *wa = reinterpret_cast<const u32x4 *>(mat + (size_t)ra * ld + col0) + lane;
    const u32x4 *wb = reinterpret_cast<const u32x4 *>(mat + (size_t)(ra + 1) * ld + col0) + lane;
#pragma unroll
    for (int i = 0; i < kAheadChunks; ++i)
        if (i < nc) {
            r.a[i] = load_stream(wa + i * 64);
            r.b[i] = load_stream(wb + i * 64);
        }
}

// Byte offset in the dynamic LDS of the 8 KiB (1 KiB per wave) that the
// opcode-6 cache warming writes into: after the SiLU staging area.
__device__ __forceinline__ uint32_t lds_prefetch_offset(kp_c &p) {
    return (uint32_t)p.F * 4u;
}

// ---------------------------------------------------------------------------
// RMSNorm + router (shared by opcodes 5 and 8)
// ---------------------------------------------------------------------------

// Expert-count specialisation: kE > 0 compiles for exactly kE experts (the
// Mixtral case, branch-free loops); kE == 0 handles any 2 <= E <= 16 at
// run time.
template <int kE>
struct Experts {
    static constexpr int kMax = kE > 0 ? kE : MK_MAX_EXPERTS;
    __device__ static __forceinline__ bool has(kp_c &p, int e) { return kE > 0 ? e < kE : e < p.E; }
};

// Per-thread norm weights and router rows, loaded before the producer wait
// (they do not depend on it), for the common case H / 8 <= threads: thread t
// owns the 8 hidden elements [8t, 8t + 8).  Threads < E also stage the router
// bias in LDS.
template <int kE>
struct RouterRegs {
    u32x4 ln;
    u32x4 rw[Experts<kE>::kMax];
};

__device__ __forceinline__ bool router_fits(kp_c &p) { return (p.H >> 3) <= kThreads; }

template <int kE>
__device__ __forceinline__ void router_prefetch(kp_c &p, SharedState &sh, int layer, const uint16_t *router,
                                                RouterRegs<kE> &rr) {
    const int v = threadIdx.x;
    if (v < p.E) sh.bias[v] = p.router_bias != nullptr ? p.router_bias[layer * p.E + v] : 0.f;
    if (!router_fits(p) || v >= (p.H >> 3)) return;
    rr.ln = reinterpret_cast<const u32x4 *>(p.ffn_ln + (size_t)layer * p.H)[v];
    const uint16_t *rw = router + (size_t)layer * p.E * p.H;
#pragma unroll
    for (int e = 0; e < Experts<kE>::kMax; ++e)
        if (Experts<kE>::has(p, e)) rr.rw[e] = reinterpret_cast<const u32x4 *>(rw + (size_t)e * p.H)[v];
}

__device__ __forceinline__ u32x4 norm8(u32x4 x, u32x4 w, float r) {
    u32x4 n;
    n.x = norm2(x.x, w.x, r);
    n.y = norm2(x.y, w.y, r);
    n.z = norm2(x.z, w.z, r);
    n.w = norm2(x.w, w.w, r);
    return n;
}

__device__ __forceinline__ float sumsq8(u32x4 x) { return sumsq2(x.x) + sumsq2(x.y) + sumsq2(x.z) + sumsq2(x.w); }

// Reduce per-thread router partials to the E logits (+ bias).  Every thread
// sums the per-wave partials itself, so the logits end up in registers after
// a single workgroup barrier.
template <int kE>
__device__ __forceinline__ void finish_logits(kp_c &p, SharedState &sh, const float *acc, float *logits) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
#pragma unroll
    for (int e = 0; e < Experts<kE>::kMax; ++e) {
        if (Experts<kE>::has(p, e)) {
            const float s = wave_sum(acc[e]);
            if (lane == 0) sh.red[e * kWaves + wave] = s;
        }
    }
    __syncthreads();
#pragma unroll
    for (int e = 0; e < Experts<kE>::kMax; ++e) {
        float s = 0.f;
        if (Experts<kE>::has(p, e)) {
#pragma unroll
            for (int i = 0; i < kWaves; ++i) s += sh.red[e * kWaves + i];
            s += sh.bias[e];
        }
        logits[e] = s;
    }
}

// normed hidden (bf16) -> act[0 .. H/8); router logits -> logits[0 .. E) in
// every thread.  Reads hidden_states, so it runs after the producer wait.
template <int kE>
__device__ __forceinline__ void rms_router(kp_c &p, SharedState &sh, u32x4 *act, int layer, const uint16_t *router,
                           const RouterRegs<kE> &rr, int32_t *tim, float *logits) {
    const int tid = threadIdx.x;
    const int nv = p.H >> 3;
    float acc[Experts<kE>::kMax];
#pragma unroll
    for (int e = 0; e < Experts<kE>::kMax; ++e) acc[e] = 0.f;

    if (router_fits(p)) {
        const bool mine = tid < nv;
        u32x4 x = {0u, 0u, 0u, 0u};
        if (mine) x = ld_dev128(p.hidden, (uint32_t)tid * 16u);
        const float sq = sumsq8(x);
        stamp(tim, 60);
        const float ss = block_sum(sq, sh.red_ss);
        stamp(tim, 61);
        const float r = 1.0f / sqrtf(ss / (float)p.H + p.eps);
        if (mine) {
            const u32x4 n = norm8(x, rr.ln, r);
            act[tid] = n;
#pragma unroll
            for (int e = 0; e < Experts<kE>::kMax; ++e)
                if (Experts<kE>::has(p, e)) acc[e] = dot8(rr.rw[e], n, 0.f);
        }
    } else {
        const u32x4 *w4 = reinterpret_cast<const u32x4 *>(p.ffn_ln + (size_t)layer * p.H);
        float ss = 0.f;
        for (int v = tid; v < nv; v += kThreads) ss += sumsq8(ld_dev128(p.hidden, (uint32_t)v * 16u));
        ss = block_sum(ss, sh.red_ss);
        const float r = 1.0f / sqrtf(ss / (float)p.H + p.eps);
        const uint16_t *rw = router + (size_t)layer * p.E * p.H;
        for (int v = tid; v < nv; v += kThreads) {
            const u32x4 n = norm8(ld_dev128(p.hidden, (uint32_t)v * 16u), w4[v], r);
            act[v] = n;
#pragma unroll
            for (int e = 0; e < Experts<kE>::kMax; ++e)
                if (Experts<kE>::has(p, e))
                    acc[e] = dot8(reinterpret_cast<const u32x4 *>(rw + (size_t)e * p.H)[v], n, acc[e]);
        }
    }
    stamp(tim, 62);
    finish_logits<kE>(p, sh, acc, logits);
    stamp(tim, 63);
}

struct Top2 {
    int i0, i1;
    float p0, p1;
};

// Top-2 of softmax(logits) in descending order, and the two probabilities.
// softmax is monotonic, so the pair is chosen on the logits (strict
// comparison: the lower expert index wins a tie); p_i = exp(l_i - max) / sum
// as torch.softmax computes it.
template <int kE>
__device__ __forceinline__ Top2 softmax_top2(kp_c &p, const float *logits) {
    int i0 = 0;
    float l0 = logits[0];
#pragma unroll
    for (int e = 1; e < Experts<kE>::kMax; ++e) {
        if (Experts<kE>::has(p, e) && logits[e] > l0) {
            i0 = e;
            l0 = logits[e];
        }
    }
    int i1 = -1;
    float l1 = 0.f;
#pragma unroll
    for (int e = 0; e < Experts<kE>::kMax; ++e) {
        if (Experts<kE>::has(p, e) && e != i0 && (i1 < 0 || logits[e] > l1)) {
            i1 = e;
            l1 = logits[e];
        }
    }
    float s = 0.f;
#pragma unroll
    for (int e = 0; e < Experts<kE>::kMax; ++e)
        if (Experts<kE>::has(p, e)) s += expf(logits[e] - l0);
    return Top2{i0, i1, 1.0f / s, expf(l1 - l0) / s};
}

// ---------------------------------------------------------------------------
// opcode 5: RmsRouterUpgate  (python_vm.py:228-277)
// ---------------------------------------------------------------------------

// Next item from the workgroup's LDS counter (uniform result).
__device__ __forceinline__ int next_local_item(SharedState &sh, int lane) {
    int v = 0;
    if (lane == 0) v = atomicAdd(&sh.next_item, 1);
    return __builtin_amdgcn_readfirstlane(v);
}

// The first of two consecutive items claimed at once.
__device__ __forceinline__ int next_local_pair(SharedState &sh, int lane) {
    int v = 0;
    if (lane == 0) v = atomicAdd(&sh.next_item, 2);
    return __builtin_amdgcn_readfirstlane(v);
}

// silu_out[e][r] = bf16(bf16(silu(bf16 g)) * bf16 u) from the wave sums of
// the gate and up rows (lane 0 stores).
__device__ __forceinline__ void silu_store(kp_c &p, int e, int r, float ag, float au, int lane) {
    if (lane == 0) {
        const float g = rbf(ag), u = rbf(au);
        const float sg = rbf(g / (1.0f + expf(-g)));
        st_dev16(p.silu + (size_t)e * p.F + r, f2bf(sg * u));
    }
}

// One item of opcode 5: row r of the FFN dimension for expert slot j, i.e.
// the gate and up rows (H bf16 each) dotted with the normed hidden state,
// then silu_out[e][r] = bf16(bf16(silu(bf16(g))) * bf16(u)).
__device__ __forceinline__ void upgate_item(kp_c &p, const u32x4 *act, int layer, int row0, int nrows,
                                            int e0, int e1, int it, int lane) {
    const int j = it >= nrows;
    const int r = row0 + (j ? it - nrows : it);
    const int e = j ? e1 : e0;
    const size_t off = ((size_t)(layer * p.E + e) * p.F + r) * (size_t)p.H;
    float ag = 0.f, au = 0.f;
    dot_pair(p.gate + off, p.up + off, act, act, p.H / kChunkElems, lane, ag, au);
    silu_store(p, e, r, wave_sum(ag), wave_sum(au), lane);
}

// Item `it` of an opcode-5 instruction when its gate and up rows are the
// ones this wave staged in LDS (the predicted top-1 expert's row row0 + it,
// staged by the preceding O projection; the loads have landed once the wave
// has waited for its own loads).
__device__ __forceinline__ void upgate_item_staged(kp_c &p, const u32x4 *act, int row0, int e, int it,
                                                   int wave, int lane) {
    const int nc = p.H / kChunkElems;
    const u32x4 *sg = act + p.stage_off16 + (wave - 1) * 2 * nc * 64 + lane, *su = sg + nc * 64;
    __builtin_amdgcn_s_waitcnt(0);
    float ag = 0.f, au = 0.f;
    for (int ch = 0; ch < nc; ++ch) {
        ag = dot8(sg[ch * 64], act[ch * 64 + lane], ag);
        au = dot8(su[ch * 64], act[ch * 64 + lane], au);
    }
    silu_store(p, e, row0 + it, wave_sum(ag), wave_sum(au), lane);
}

// Wave-level claim of the next item of an instruction.  Lane 0 issues the
// atomic; the value is broadcast only where it is needed, so the wait for the
// atomic's return can sit behind the current item's weight loads.
__device__ __forceinline__ int claim_issue(int32_t *cursor, int lane) {
    int v = 0;
    if (lane == 0) v = __hip_atomic_fetch_add(cursor, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    return v;
}

// Wave 0 collects the group's opcode-5 instructions of `layer` (workers
// [group * kPoolGroup, +kPoolGroup)) into sh.pool_*, in (worker, slot)
// order, looking at the queue slots [slot - kPoolWindow / 2, +kPoolWindow)
// of each member: the instructions of one layer sit at about the same queue
// depth on every worker, and this way one round trip reads all of them
// (wave 0 has no staging loads in flight ahead of it).  An instruction
// outside the window is only left out of the sharing (its owner still does
// all of its items); out-of-range operands are left out too (their owner
// reports them).  The caller's next workgroup barrier publishes the pool.
__device__ __forceinline__ void pool_scan_near(kp_c &p, SharedState &sh, int layer, int group, int slot) {
    static_assert(kPoolGroup * kPoolWindow == 64, "pool_scan_near: one slot per lane of wave 0");
    const int lane = threadIdx.x & 63;
    const int w0 = group * kPoolGroup, mate = lane / kPoolWindow;
    const int q = max(0, slot - kPoolWindow / 2) + lane % kPoolWindow;
    int4 wd = make_int4(0, 0, 0, 0);
    if (w0 + mate < (int)gridDim.x && q < p.queue_len)
        wd = *reinterpret_cast<const int4 *>(p.instructions +
                                             ((size_t)(w0 + mate) * p.queue_len + q) * MK_INTS_PER_INSTRUCTION);
    const int start = wd.z, nb = wd.w;
    const bool m = wd.x == 5 && wd.y == layer && start >= 0 && nb > 0 &&
                   (int64_t)(start + nb) * p.expert_bs <= (int64_t)p.F;
    const uint64_t bal = __ballot(m);
    if (m) {
        const int k = __popcll(bal & ((1ull << lane) - 1ull));
        sh.pool_slot[k] = (w0 + mate) * p.queue_len + q;
        sh.pool_row0[k] = start * p.expert_bs;
        sh.pool_nrows[k] = nb * p.expert_bs;
    }
    if (lane == 0) sh.pool_n = __popcll(bal);
}

__device__ __forceinline__ int tail_items(kp_c &p, int items) { return items < p.tail_items ? items : p.tail_items; }

__device__ __forceinline__ int32_t *slot_cursor(kp_c &p, int slot) {
    return p.scratch + kScratchSlotBase + 2 * slot;
}

// Items [first, first + count) of an opcode-5 instruction whose FFN rows
// start at row0 (nrows rows, items 0 .. 2*nrows), claimed one at a time from
// the instruction's cursor (the next claim is issued before the current
// item's loads) until the cursor passes count.  Returns the number done here.
__device__ __forceinline__ int upgate_claimed(kp_c &p, const u32x4 *act, int layer, int row0, int nrows, int e0, int e1,
                              int first, int count, int32_t *cursor, int lane) {
    int done_here = 0;
    int c = __builtin_amdgcn_readfirstlane(claim_issue(cursor, lane));
    while (c < count) {
        int next_raw = claim_issue(cursor, lane);
        upgate_item(p, act, layer, row0, nrows, e0, e1, first + c, lane);
        ++done_here;
        // first use of the claim result: keeps the compiler from hoisting the
        // broadcast (and the wait for the atomic) above the item's loads
        asm volatile("" : "+v"(next_raw));
        c = __builtin_amdgcn_readfirstlane(next_raw);
    }
    return done_here;
}

// A wave reports `n` finished items of an instruction (after its own stores
// have completed).  The owner's report carries one extra count, so an
// instruction completes only after its owner has also published the routing
// (for the block-0 instruction); the report that reaches items + 1 arrives
// for the instruction's rows on the layer and chunk counters.
__device__ __forceinline__ void publish_items(kp_c &p, int32_t *done, int n, int items, int row0,
                                              int nrows, int layer, int lane) {
    if (n <= 0) return;
    __builtin_amdgcn_s_waitcnt(0);
    if (lane == 0) {
        const int prev = __hip_atomic_fetch_add(done, n, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (prev + n == items + 1) arrive_add(p, bar_at(p, layer, 5), nrows / p.expert_bs);
    }
}

// After its own instruction, each wave takes unclaimed tail items of the
// other group instructions: one vector load reads every cursor, the wave
// picks the first instruction with items left (starting at an offset that
// spreads the waves), claims from it until it is exhausted, and repeats.
// Routing is a function of the layer's inputs only, so the experts are the
// owner's.
__device__ __forceinline__ void steal_upgate(kp_c &p, const SharedState &sh, const u32x4 *act, int layer, int self_k,
                             int e0, int e1, int lane, int wave) {
    const int n = sh.pool_n;
    const int start = (self_k + 1 + wave) % n;
    for (;;) {
        int left = 0;
        if (lane < n && lane != self_k) {
            const int tail = tail_items(p, 2 * sh.pool_nrows[lane]);
            left = tail - (int)ld_dev32(slot_cursor(p, sh.pool_slot[lane]));
        }
        uint64_t b = __ballot(left > 0);
        if (b == 0) break;
        // first candidate at or after `start`, wrapping around
        const uint64_t hi = b >> start;
        const int v = hi != 0 ? start + (int)__builtin_ctzll(hi) : (int)__builtin_ctzll(b);
        const int nrows = sh.pool_nrows[v], items = 2 * nrows, tail = tail_items(p, items);
        int32_t *cursor = slot_cursor(p, sh.pool_slot[v]);
        const int got = upgate_claimed(p, act, layer, sh.pool_row0[v], nrows, e0, e1, items - tail, tail, cursor, lane);
        publish_items(p, cursor + 1, got, items, sh.pool_row0[v], nrows, layer, lane);
    }
}

// Count a finished item of pooled instruction k (lane 0; the wave's SiLU
// stores of it have completed).  The item that completes the instruction
// arrives for its blocks on the layer counter and, with the overlap on, adds
// its rows to the column-chunk counters.
__device__ __forceinline__ void upgate_item_done(kp_c &p, SharedState &sh, int layer, int k, int lane) {
    if (lane != 0 || k < 0) return;
    const int r0 = sh.grp_row0[k], n = sh.grp_nrows[k];
    if (atomicAdd(&sh.grp_done[k], 1) + 1 != 2 * n) return;
    arrive_add(p, bar_at(p, layer, 5), n / p.expert_bs);
    if (p.chunk_ctr != nullptr) {
        int32_t *cc = p.chunk_ctr + (size_t)layer * (p.F / kChunkElems);
        for (int r = r0; r < r0 + n;) {
            const int ch = r / kChunkElems, e = min(r0 + n, (ch + 1) * kChunkElems);
            __hip_atomic_fetch_add(cc + ch, e - r, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            r = e;
        }
    }
}

// `consumed` returns the queue slots handled: without work sharing, the
// instructions of the same layer that follow this one in the worker's queue
// (kMaxMerge at most) run as one pool of items, so the routing is computed
// once and no wave waits for another between them.
template <int kE, bool kSpec>
__device__ __forceinline__ bool op_rms_router_upgate(kp_c &p, SharedState &sh, u32x4 *act, ins_t *ins,
                                                     const Ctx &c, int32_t *tim, int &consumed) {
    const int layer = __builtin_amdgcn_readfirstlane(ins[1]);
    const int start = __builtin_amdgcn_readfirstlane(ins[2]);
    const int nb = __builtin_amdgcn_readfirstlane(ins[3]);
    consumed = 1;
    if (layer < 0 || layer >= p.num_layers || start < 0 || nb < 0 ||
        (int64_t)(start + nb) * p.expert_bs > (int64_t)p.F) {
        report_error(p, MK_ERR_BAD_INSTRUCTION, c, 5, layer, start, nb);
        return false;
    }
    // an empty instruction owns no rows (another one starts at block 0)
    if (nb == 0) return true;
    int K = 1;
    bool pub = start == 0;  // the pool holds the instruction that starts at block 0
    if (!p.work_sharing) {
        // the next kMaxMerge - 1 slots' words, read without a dependency
        // between them (slot indices clamped to the queue: one round trip);
        // whole-model kernels (kSpec) run one instruction at a time, which
        // keeps their registers within the budget
        constexpr int kPool = kSpec ? 1 : kMaxMerge;
        int st_k[kPool], nb_k[kPool];
        bool more = true;
        st_k[0] = start;
        nb_k[0] = nb;
#pragma unroll
        for (int k = 1; k < kPool; ++k) {
            ins_t *n = ins + (min(c.slot + k, p.queue_len - 1) - c.slot) * MK_INTS_PER_INSTRUCTION;
            const int op_n = __builtin_amdgcn_readfirstlane(n[0]);
            const int layer_n = __builtin_amdgcn_readfirstlane(n[1]);
            st_k[k] = __builtin_amdgcn_readfirstlane(n[2]);
            nb_k[k] = __builtin_amdgcn_readfirstlane(n[3]);
            // an out-of-range instruction ends the pool and reports itself
            more = more && c.slot + k < p.queue_len && op_n == 5 && layer_n == layer && st_k[k] >= 0 &&
                   nb_k[k] > 0 && (int64_t)(st_k[k] + nb_k[k]) * p.expert_bs <= (int64_t)p.F;
            if (more) {
                pub = pub || st_k[k] == 0;
                ++K;
            }
        }
        if (threadIdx.x == 0) {
            int first = 0;
#pragma unroll
            for (int k = 0; k < kPool; ++k) {
                if (k < K) {
                    sh.grp_row0[k] = st_k[k] * p.expert_bs;
                    sh.grp_nrows[k] = nb_k[k] * p.expert_bs;
                    sh.grp_first[k] = first;
                    sh.grp_done[k] = 0;
                    first += 2 * nb_k[k] * p.expert_bs;
                }
            }
            sh.grp_first[K] = first;
        }
    } else if (threadIdx.x == 0) {
        // work sharing: a pool of this instruction alone, which the static
        // path below uses when the group has more instructions than the
        // shared pool can list
        sh.grp_row0[0] = start * p.expert_bs;
        sh.grp_nrows[0] = nb * p.expert_bs;
        sh.grp_first[0] = 0;
        sh.grp_first[1] = 2 * nb * p.expert_bs;
        sh.grp_done[0] = 0;
    }
    consumed = K;
    auto wait = [&] { return wait_ge(p, sh, bar_at(p, layer, 4), p.H / p.oproj_bs, c, 5, layer); };
    if (kSpec && p.late_loads && !wait()) return false;  // whole-model launches only
    // the pool's instruction list does not depend on the producers either
    // (the wait below, or rms_router's, is the workgroup barrier after it)
    if (p.work_sharing && __builtin_amdgcn_readfirstlane(threadIdx.x >> 6) == 0)
        pool_scan_near(p, sh, layer, c.worker / kPoolGroup, c.slot);
    RouterRegs<kE> rr;
    router_prefetch<kE>(p, sh, layer, p.router, rr);
    // items 0 .. kWaves-1 go to waves 0 .. kWaves-1, the rest through the
    // LDS counter (reset here; the wait below is a workgroup barrier)
    if (threadIdx.x == 0) sh.next_item = kWaves;
    const int row0 = start * p.expert_bs, nrows = nb * p.expert_bs;
    // Speculative early loads (whole-model launches): the preceding O
    // projection may have staged this instruction's first items of the
    // predicted top-1 expert in LDS (stage_moe_upgate).  Staging them here
    // instead, at the start of opcode 5, gained nothing: 256 workgroups then
    // load 28 MB at the moment the O projection hands over, which delays
    // every workgroup's detection of that hand-off by ~4 us.
    int staged = 0;  // items 1 .. staged of this instruction are in LDS (of expert spec_e[0])
    if constexpr (kSpec && kE > 0) {
        if (threadIdx.x == 0) {
            if (sh.stage_slot != c.slot) {
                // the prediction only for the timing record
                int e0 = -1, e1 = -1;
                if (tim != nullptr && !p.work_sharing) {
                    const int32_t *pc = bar_at(p, layer, 8);
                    if (counter_value(p, pc, spread_row(p, pc)) >= 1) {
                        e0 = (int)ld_dev32(p.pred_idx);
                        e1 = (int)ld_dev32(p.pred_idx + 1);
                    }
                }
                sh.spec_e[0] = e0;
                sh.spec_e[1] = e1;
            } else if (tim != nullptr) {
                sh.spec_e[1] = (int)ld_dev32(p.pred_idx + 1);
            }
        }
        __syncthreads();
        staged = __builtin_amdgcn_readfirstlane(sh.stage_slot == c.slot ? sh.stage_n : 0);
        if (staged > 0) stamp(tim, MK_TEVENT_FIRST_USE);
    }
    stamp(tim, MK_TEVENT_AT_GMEM_WAIT);
    if (!(kSpec && p.late_loads) && !wait()) return false;
    stamp(tim, MK_TEVENT_DONE_GMEM_WAIT);

    float logits[Experts<kE>::kMax];
    rms_router<kE>(p, sh, act, layer, p.router, rr, tim, logits);
    const Top2 t = softmax_top2<kE>(p, logits);
    if constexpr (kSpec) {
        // predicted and selected experts, one byte each (0xff: no prediction)
        if (tim != nullptr && threadIdx.x == 0)
            tim[MK_TEVENT_PREDICTION] = (int32_t)((uint32_t)(sh.spec_e[0] & 0xff) | ((uint32_t)(sh.spec_e[1] & 0xff) << 8) |
                                                  ((uint32_t)t.i0 << 16) | ((uint32_t)t.i1 << 24));
    }
    const float psum = t.p0 + t.p1;
    const uint32_t sc0 = f2bf(t.p0 / psum), sc1 = f2bf(t.p1 / psum);
    const int tid = threadIdx.x;
    if (tid == 0) {
        sh.route_layer = layer;
        sh.route_idx[0] = t.i0;
        sh.route_idx[1] = t.i1;
        sh.route_score[0] = bf2f(sc0);
        sh.route_score[1] = bf2f(sc1);
    }
    // Exactly one instruction per layer starts at block 0: it publishes the
    // normed hidden state and the routing decision.
    if (pub) {
        u32x4 *out = reinterpret_cast<u32x4 *>(p.normed_out);
        for (int v = tid; v < (p.H >> 3); v += kThreads) st_dev128(out + v, act[v]);
        if (tid == 0) {
            st_dev32(p.sel_idx, (uint32_t)t.i0);
            st_dev32(p.sel_idx + 1, (uint32_t)t.i1);
            st_dev16(p.sel_score, sc0);
            st_dev16(p.sel_score + 1, sc1);
        }
        // items complete (and arrive) one wave at a time, and a wave may do
        // none: every wave's part of the publication completes first
        drain_and_sync();
    }
    stamp(tim, MK_TEVENT_FIRST_LOAD);

    const int lane = tid & 63, wave = tid >> 6;
    if (p.work_sharing && sh.pool_n <= kMaxPoolIns) {
        // Own items first: all but the tail from the LDS counter, the tail
        // through this instruction's cursor; then the group's leftovers.  No
        // worker waits for another: whoever completes an instruction's items
        // arrives for it.
        const int self_slot = c.worker * p.queue_len + c.slot;
        int self_k = 0;
        while (self_k < sh.pool_n - 1 && sh.pool_slot[self_k] != self_slot) ++self_k;
        int32_t *cursor = slot_cursor(p, self_slot);
        const int items = 2 * nrows, tail = tail_items(p, items);
        // a wave's first item (item `wave`) may be staged in LDS, as in the
        // static path below
        const bool from_lds = kSpec && kE > 0 && staged > 0 && wave >= 1 && wave <= staged && wave < nrows &&
                              __builtin_amdgcn_readfirstlane(sh.spec_e[0]) == t.i0;
        int mine = 0;
        for (int it = wave; it < items - tail; it = next_local_item(sh, lane)) {
            if (kSpec && kE > 0 && mine == 0 && from_lds)
                upgate_item_staged(p, act, row0, t.i0, it, wave, lane);
            else
                upgate_item(p, act, layer, row0, nrows, t.i0, t.i1, it, lane);
            ++mine;
        }
        mine += upgate_claimed(p, act, layer, row0, nrows, t.i0, t.i1, items - tail, tail, cursor, lane);
        // wave 0 also carries the owner's extra count
        publish_items(p, cursor + 1, mine + (wave == 0), items, row0, nrows, layer, lane);
        stamp(tim, MK_TEVENT_AT_GMEM_STORE);
        if (sh.pool_n > 1) steal_upgate(p, sh, act, layer, self_k, t.i0, t.i1, lane, wave);
        drain_and_sync();
        stamp(tim, MK_TEVENT_DONE_GMEM_STORE);
    } else {
        // Waves take items from a workgroup counter in LDS rather than a
        // fixed stride: the memory pipeline favours older waves, so with a
        // fixed split the youngest wave ends up finishing its last items
        // alone.  An item is counted once the next one's weights have been
        // used: its SiLU store has then completed (a wait for it costs
        // nothing there), so no wave stops streaming to publish rows.
        const int total = __builtin_amdgcn_readfirstlane(sh.grp_first[K]);
        // the staged items hold the predicted top-1 expert's rows: usable if
        // the routing picked it first (items 0 .. nrows-1 are slot 0)
        const bool from_lds = kSpec && kE > 0 && staged > 0 && wave >= 1 && wave <= staged &&
                              __builtin_amdgcn_readfirstlane(sh.spec_e[0]) == t.i0;
        int k = 0, pending = -1;
        for (int it = wave; it < total; ++k) {
            int q = 0;
            while (q + 1 < K && it >= __builtin_amdgcn_readfirstlane(sh.grp_first[q + 1])) ++q;
            const int local = it - __builtin_amdgcn_readfirstlane(sh.grp_first[q]);
            const int r0 = __builtin_amdgcn_readfirstlane(sh.grp_row0[q]);
            const int nr = __builtin_amdgcn_readfirstlane(sh.grp_nrows[q]);
            const int j = local >= nr;
            const int r = r0 + (j ? local - nr : local);
            const int e = j ? t.i1 : t.i0;
            float ag = 0.f, au = 0.f;
            if (kSpec && kE > 0 && k == 0 && from_lds) {
                // this wave's own staged rows (its loads have landed: it has
                // waited for its hidden-state loads since)
                const int nc = p.H / kChunkElems;
                const u32x4 *sg = act + p.stage_off16 + (wave - 1) * 2 * nc * 64 + lane, *su = sg + nc * 64;
                __builtin_amdgcn_s_waitcnt(0);
                for (int ch = 0; ch < nc; ++ch) {
                    ag = dot8(sg[ch * 64], act[ch * 64 + lane], ag);
                    au = dot8(su[ch * 64], act[ch * 64 + lane], au);
                }
            } else {
                const size_t off = ((size_t)(layer * p.E + e) * p.F + r) * (size_t)p.H;
                dot_pair(p.gate + off, p.up + off, act, act, p.H / kChunkElems, lane, ag, au);
            }
            ag = wave_sum(ag);
            au = wave_sum(au);
            __builtin_amdgcn_s_waitcnt(0);
            upgate_item_done(p, sh, layer, pending, lane);
            silu_store(p, e, r, ag, au, lane);
            pending = q;
            // per-item completion times of waves 0 and 7 (timing record only)
            if (tim != nullptr && lane == 0 && (wave == 0 || wave == kWaves - 1) && k < 16)
                tim[64 + (wave ? 16 : 0) + k] = (int32_t)(uint32_t)__builtin_amdgcn_s_memrealtime();
            it = next_local_item(sh, lane);
        }
        __builtin_amdgcn_s_waitcnt(0);
        upgate_item_done(p, sh, layer, pending, lane);
        drain_and_sync();
        stamp(tim, MK_TEVENT_DONE_GMEM_STORE);
        // the pooled slots share this one's times (one stream of items over
        // the same window, so each slot's bytes are spread over it)
        if (tim != nullptr && threadIdx.x == 0)
            for (int m = 1; m < K; ++m) {
                int32_t *tm = tim + m * MK_TIMING_SLOTS;
                for (const int ev : {MK_TEVENT_START, MK_TEVENT_AT_GMEM_WAIT, MK_TEVENT_DONE_GMEM_WAIT,
                                     MK_TEVENT_FIRST_LOAD, MK_TEVENT_DONE_GMEM_STORE})
                    tm[ev] = tim[ev];
                tm[MK_TEVENT_END] = (int32_t)(uint32_t)__builtin_amdgcn_s_memrealtime();
            }
    }
    return true;
}


// ---------------------------------------------------------------------------
// opcode 6: ExpertDownProjFused  (python_vm.py:284-314)
// ---------------------------------------------------------------------------

// Up to N chunks (512 bf16 each) of one row, n of them used (n uniform).
template <int N>
struct RowRegs {
    u32x4 w[N];
};

template <int N>
__device__ __forceinline__ void load_row(RowRegs<N> &r, const u32x4 *w, int n) {
#pragma unroll
    for (int i = 0; i < N; ++i)
        if (i < n) r.w[i] = load_stream(w + i * 64);
}

template <int N>
__device__ __forceinline__ float dot_row_regs(const RowRegs<N> &r, const u32x4 *x, int n, float acc) {
#pragma unroll
    for (int i = 0; i < N; ++i)
        if (i < n) acc = dot8(r.w[i], x[i * 64], acc);
    return acc;
}

constexpr int kSegChunks = 16;   // chunks a dense down-projection wave loads at a time (16 KiB)
constexpr int kRowBatch = kRowBatchLds;

struct DownItem {
    int row, slot, c0, n;  // batch-relative row, expert slot, first chunk, chunks
};

// Item `it` of a batch: row it / (2 S), expert slot (it / S) % 2, segment
// it % S of a row split into S segments of nc / S (+1) chunks.
__device__ __forceinline__ DownItem down_item(int it, int S, int nc) {
    const int seg = it % S;
    const int c0 = seg * nc / S, c1 = (seg + 1) * nc / S;
    return DownItem{it / (2 * S), (it / S) & 1, c0, c1 - c0};
}

// Opcode 6 streams its items through two register sets: while one item's
// partial dot is formed, the next item's loads are in flight, so a wave
// keeps one to two items (7-14 KiB) of loads outstanding instead of one
// draining to none -- the bytes in flight per compute unit are what bound
// its share of the memory bandwidth.  An item always issues kPipeChunks
// loads (an item of fewer chunks loads its last chunk again), so the
// compiler can count the loads still outstanding after each one and wait
// for one register set only; 7 chunks is Mixtral's exact segment (14336
// columns = 4 x 7 x 512).
constexpr int kPipeChunks = 7;  // chunks per opcode-6 item (7 KiB per wave)
constexpr int kVmcntZero = 0x0F70;  // s_waitcnt vmcnt(0), expcnt and lgkmcnt not waited on
static_assert(kMaxSegments * kPipeChunks * kChunkElems >= kMaxIntermediate, "opcode-6 segments cover F");

// Issues the loads of item `it` (rows [row0b, ...) of the batch) into r.
__device__ __forceinline__ void down_item_load(kp_c &p, RowRegs<kPipeChunks> &r, int it, int S, int nc,
                                               size_t base0, size_t base1, int row0b, int lane) {
    const DownItem d = down_item(it, S, nc);
    const uint16_t *row = p.down + ((d.slot ? base1 : base0) + row0b + d.row) * (size_t)p.F;
    const u32x4 *w = reinterpret_cast<const u32x4 *>(row) + d.c0 * 64 + lane;
#pragma unroll
    for (int i = 0; i < kPipeChunks; ++i) r.w[i] = load_stream(w + min(i, d.n - 1) * 64);
}

// The partial dot of item `it` (loaded into r) with the staged SiLU row of
// its expert slot, to sh.part[row][slot][segment].
__device__ __forceinline__ void down_item_finish(SharedState &sh, const RowRegs<kPipeChunks> &r, const u32x4 *act,
                                                 int nv, int it, int S, int nc, int lane) {
    const DownItem d = down_item(it, S, nc);
    const u32x4 *x = act + (d.slot ? nv : 0) + d.c0 * 64 + lane;
    float acc = 0.f;
#pragma unroll
    for (int i = 0; i < kPipeChunks; ++i) {  // straight-line: chunks past d.n (reloads) are dropped
        const float t = dot8(r.w[i], x[min(i, d.n - 1) * 64], acc);
        acc = i < d.n ? t : acc;
    }
    acc = wave_sum(acc);
    if (lane == 0) sh.part[(d.row * 2 + d.slot) * kMaxSegments + (it % S)] = acc;
}

// Opcode 6 overlapped with the end of opcode 5 (chunk counters on, and this
// workgroup routed the layer itself, so the experts are known).  The SiLU
// columns are taken in fixed groups of kGroupChunks 512-column chunks: as
// soon as every row of a group is final (its chunk counters are full), the
// group's SiLU values are staged in LDS and the instruction's rows are dotted
// with them, a row pair and both experts per item (16 loads per lane in
// flight).  The partial sum of each (row, expert, group) goes to LDS, and
// the row's total is summed over the groups in a fixed order, so the result
// does not depend on when a group became ready.
__device__ __forceinline__ bool downproj_overlapped(kp_c &p, SharedState &sh, u32x4 *act, const Ctx &c,
                                                    int32_t *tim, int layer, int start, int end) {
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int row0 = start * p.down_bs, nrows = (end - start) * p.down_bs;
    const int nc = p.F / kChunkElems;
    const int ng = (nc + kGroupChunks - 1) / kGroupChunks;
    const int nv = p.F >> 3;
    const int npairs = nrows / kItemRows;
    const int e0 = sh.route_idx[0], e1 = sh.route_idx[1];
    const float s0 = sh.route_score[0], s1 = sh.route_score[1];
    // opcode 5 ran here, after the O-projection barrier: the residual rows
    // are final
    uint32_t hpre = 0;
    if (tid < nrows) hpre = ld_dev16(p.hidden + row0 + tid);
    const int32_t *cc = p.chunk_ctr + (size_t)layer * nc;
    const uint16_t *a0 = p.silu + (size_t)e0 * p.F;
    const uint16_t *a1 = p.silu + (size_t)e1 * p.F;
    const uint16_t *w0 = p.down + ((size_t)(layer * p.E + e0) * p.H + row0) * (size_t)p.F;
    const uint16_t *w1 = p.down + ((size_t)(layer * p.E + e1) * p.H + row0) * (size_t)p.F;
    const uint32_t all = (1u << ng) - 1u;
    uint32_t done = 0;
    stamp(tim, MK_TEVENT_AT_GMEM_WAIT);
    while (done != all) {
        // thread 0 polls until a group not yet done is complete
        if (tid == 0) {
            uint32_t ready = 0;
            int ok = 1, nap = 1;
            uint64_t t0 = 0;
            for (;;) {
                for (int g = 0; g < ng; ++g) {
                    if ((done >> g) & 1u) continue;
                    bool full = true;
                    for (int k = 0; k < kGroupChunks; ++k) {
                        const int ch = g * kGroupChunks + k;
                        if (ch < nc && (int)ld_dev32(cc + ch) < kChunkElems) full = false;
                    }
                    if (full) ready |= 1u << g;
                }
                if (ready != 0) break;
                if (aborted(p)) {
                    ok = 0;
                    break;
                }
                const uint64_t now = __builtin_amdgcn_s_memrealtime();
                if (t0 == 0) {
                    t0 = now;
                } else if (now - t0 > (uint64_t)p.timeout_ticks) {
                    report_error_lane(p, MK_ERR_TIMEOUT, c, 6, layer, (int)all, (int)done);
                    ok = 0;
                    break;
                }
                for (int i = 0; i < nap; ++i) __builtin_amdgcn_s_sleep(1);
                if (nap < p.spin_max) nap *= 2;
            }
            sh.ready_mask = ok ? (int)ready : -1;
        }
        __syncthreads();
        const int rm = __builtin_amdgcn_readfirstlane(sh.ready_mask);
        if (rm < 0) return false;
        const uint32_t fresh = (uint32_t)rm;
        // the fresh groups' SiLU values of both experts, at their offsets
        for (int v = tid; v < nv; v += kThreads) {
            if ((fresh >> ((v >> 6) / kGroupChunks)) & 1u) {
                act[v] = ld_dev128(a0, (uint32_t)v * 16u);
                act[nv + v] = ld_dev128(a1, (uint32_t)v * 16u);
            }
        }
        if (tid == 0) sh.next_item = kWaves;
        __syncthreads();
        const int items = __popc(fresh) * npairs;
        for (int it = wave; it < items; it = next_local_item(sh, lane)) {
            uint32_t m = fresh;
            for (int k = it / npairs; k > 0; --k) m &= m - 1u;
            const int g = __builtin_ctz(m);
            const int pr = it % npairs;
            const int c0 = g * kGroupChunks, n = min(kGroupChunks, nc - c0);
            // i = 0 .. 2 kItemRows - 1: row kItemRows pr + (i >> 1) of expert slot i & 1
            const size_t roff = (size_t)(kItemRows * pr) * p.F + (size_t)(c0 * kChunkElems + lane * 8);
            u32x4 w[2 * kItemRows][kGroupChunks];
#pragma unroll
            for (int i = 0; i < 2 * kItemRows; ++i) {
                const u32x4 *rw = reinterpret_cast<const u32x4 *>(((i & 1) ? w1 : w0) + roff + (i >> 1) * (size_t)p.F);
                // a short last group loads its last chunk again in place of the
                // missing ones and drops them from the sums (selects, no
                // branches: conditional loads here put the array in scratch)
#pragma unroll
                for (int k = 0; k < kGroupChunks; ++k) w[i][k] = load_stream(rw + min(k, n - 1) * 64);
            }
            float acc[2 * kItemRows];
#pragma unroll
            for (int i = 0; i < 2 * kItemRows; ++i) {
                const u32x4 *x = act + ((i & 1) ? nv : 0) + c0 * 64 + lane;
                acc[i] = 0.f;
#pragma unroll
                for (int k = 0; k < kGroupChunks; ++k) {
                    const float d = dot8(w[i][k], x[min(k, n - 1) * 64], 0.f);
                    acc[i] += k < n ? d : 0.f;
                }
                acc[i] = wave_sum(acc[i]);
            }
            if (lane == 0) {
#pragma unroll
                for (int i = 0; i < 2 * kItemRows; ++i)
                    sh.part[((kItemRows * pr + (i >> 1)) * 2 + (i & 1)) * kMaxGroups + g] = acc[i];
            }
        }
        __syncthreads();
        done |= fresh;
    }
    stamp(tim, MK_TEVENT_DONE_GMEM_WAIT);
    // the reference's condition (every opcode-5 block arrived) holds by now
    // or within a few polls: the chunk counters are added after it
    if (!wait_ge(p, sh, bar_at(p, layer, 5), p.F / p.expert_bs, c, 6, layer)) return false;
    stamp(tim, MK_TEVENT_FIRST_LOAD);
    // h = bf16(h + bf16(s_j * bf16(d_j))) for j = 0, 1 in order
    for (int r = tid; r < nrows; r += kThreads) {
        float d0 = 0.f, d1 = 0.f;
        for (int g = 0; g < ng; ++g) {
            d0 += sh.part[(r * 2 + 0) * kMaxGroups + g];
            d1 += sh.part[(r * 2 + 1) * kMaxGroups + g];
        }
        float h = bf2f(hpre);  // r == tid: nrows <= kThreads
        h = rbf(h + rbf(s0 * rbf(d0)));
        h = rbf(h + rbf(s1 * rbf(d1)));
        st_dev16(p.hidden + row0 + r, f2bf(h));
    }
    drain_and_sync();
    arrive(p, bar_at(p, layer, 6), 2 * (end - start));
    stamp(tim, MK_TEVENT_DONE_GMEM_STORE);
    return true;
}

// kOverlap: the overlapped form is compiled in (the 8-expert MoE-only
// kernel; in the others its registers would spill).
template <bool kOverlap>
__device__ __forceinline__ bool op_expert_downproj(kp_c &p, SharedState &sh, u32x4 *act, ins_t *ins,
                                   const Ctx &c, int32_t *tim) {
    const int layer = __builtin_amdgcn_readfirstlane(ins[1]);
    const int start = __builtin_amdgcn_readfirstlane(ins[2]);
    const int end = __builtin_amdgcn_readfirstlane(ins[3]);
    const int red = __builtin_amdgcn_readfirstlane(ins[4]);
    if (layer < 0 || layer >= p.num_layers || start < 0 || end < start ||
        (int64_t)end * p.down_bs > (int64_t)p.H || red != 0) {
        report_error(p, MK_ERR_BAD_INSTRUCTION, c, 6, layer, start, end);
        return false;
    }
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int row0 = start * p.down_bs, nrows = (end - start) * p.down_bs;
    const int nc = p.F / kChunkElems;
    const int S = (nc + kPipeChunks - 1) / kPipeChunks;  // column segments per row

    // Early loads: when this workgroup routed the layer itself (opcode 5 ran
    // here), the experts are known before the barrier, so each wave starts
    // streaming its two first items (wave and wave + 8) while it waits.
    const bool known = !(!kOverlap && p.late_loads) && sh.route_layer == layer;  // late loads: whole-model only
    if (kOverlap && p.chunk_ctr != nullptr && known && nrows <= 32 && nrows % kItemRows == 0 && (p.F % kChunkElems) == 0 &&
        nc <= kGroupChunks * kMaxGroups)
        return downproj_overlapped(p, sh, act, c, tim, layer, start, end);
    const int first_batch = min(nrows, kRowBatch);
    const bool early = known && p.early_loads != 0;
    RowRegs<kPipeChunks> A, B;
    if (early) {
        const size_t k0 = (size_t)(layer * p.E + sh.route_idx[0]) * p.H;
        const size_t k1 = (size_t)(layer * p.E + sh.route_idx[1]) * p.H;
        if (wave < first_batch * 2 * S) down_item_load(p, A, wave, S, nc, k0, k1, row0, lane);
        if (wave + kWaves < first_batch * 2 * S) down_item_load(p, B, wave + kWaves, S, nc, k0, k1, row0, lane);
    }
    // The residual rows this instruction updates: when opcode 5 ran here,
    // the O-projection barrier it waited for has made them final, so they
    // are read now instead of after the sums (one dependent load less).
    uint32_t hpre = 0;
    if (known && tid < first_batch) hpre = ld_dev16(p.hidden + row0 + tid);

    stamp(tim, MK_TEVENT_AT_GMEM_WAIT);
    int32_t *ready = bar_at(p, layer, 5);
    const int expected = p.F / p.expert_bs;
    // Cache warming: if opcode 5 is still running elsewhere, HBM has spare
    // bandwidth, so each wave reads the rows of its next items once more
    // with ordinary (cache-allocating) loads straight into a scratch corner
    // of LDS; after the wait, their regular loads find them in the
    // Infinity Cache.  Workgroups that arrive after the last producer skip
    // it.
    if (known && p.pf_rounds > 0) {
        const bool warm = !counter_reached(p, sh, ready, expected);
        if (warm) {
            __attribute__((address_space(3))) void *sink =
                (__attribute__((address_space(3))) void *)(act + (lds_prefetch_offset(p) >> 4) + wave * 64);
            for (int m = 1; m <= p.pf_rounds; ++m) {
                const int it = wave + (m + 1) * kWaves;  // the items after the wave's two first
                if (it >= first_batch * 2 * S) break;
                const DownItem d = down_item(it, S, nc);
                const int e = sh.route_idx[d.slot];
                const uint16_t *row = p.down + ((size_t)(layer * p.E + e) * p.H + row0 + d.row) * (size_t)p.F;
                const u32x4 *w = reinterpret_cast<const u32x4 *>(row) + d.c0 * 64 + lane;
                for (int i = 0; i < d.n; ++i)
                    __builtin_amdgcn_global_load_lds((const __attribute__((address_space(1))) void *)(w + i * 64),
                                                     sink, 16, 0, 0);
            }
        }
    }
    if (!wait_ge(p, sh, ready, expected, c, 6, layer)) return false;
    stamp(tim, MK_TEVENT_DONE_GMEM_WAIT);

    int e0, e1;
    float s0, s1;
    if (known) {
        e0 = sh.route_idx[0];
        e1 = sh.route_idx[1];
        s0 = sh.route_score[0];
        s1 = sh.route_score[1];
    } else {
        e0 = __builtin_amdgcn_readfirstlane((int)ld_dev32(p.sel_idx));
        e1 = __builtin_amdgcn_readfirstlane((int)ld_dev32(p.sel_idx + 1));
        s0 = bf2f(ld_dev16(p.sel_score));
        s1 = bf2f(ld_dev16(p.sel_score + 1));
    }
    if (e0 < 0 || e0 >= p.E || e1 < 0 || e1 >= p.E) {
        report_error(p, MK_ERR_BAD_INSTRUCTION, c, 6, layer, e0, e1);
        return false;
    }

    const int nv = p.F >> 3;
    const uint16_t *a0 = p.silu + (size_t)e0 * p.F;
    const uint16_t *a1 = p.silu + (size_t)e1 * p.F;
    for (int v = tid; v < nv; v += kThreads) {
        act[v] = ld_dev128(a0, (uint32_t)v * 16u);
        act[nv + v] = ld_dev128(a1, (uint32_t)v * 16u);
    }
    if (tid == 0) sh.next_item = 2 * kWaves;
    __syncthreads();
    stamp(tim, MK_TEVENT_FIRST_LOAD);
    // Every load issued so far has landed (the early ones before the
    // barrier polls, the activations before their LDS stores); saying so
    // lets the compiler count the pipeline's outstanding loads exactly.
    __builtin_amdgcn_s_waitcnt(kVmcntZero);

    const size_t base0 = (size_t)(layer * p.E + e0) * p.H;
    const size_t base1 = (size_t)(layer * p.E + e1) * p.H;
    for (int b0 = 0; b0 < nrows; b0 += kRowBatch) {
        const int nb_rows = min(kRowBatch, nrows - b0);
        const int items = nb_rows * 2 * S;
        // items wave and wave + kWaves first (loaded early in the first
        // batch), then pairs of consecutive items claimed from the LDS
        // counter (items is even, so a pair below items lies wholly in the
        // batch; claims only grow, so the first one past it ends the
        // loop).  At the loop head A's item, then B's, are loaded or in
        // flight, in that order, and the loop's only exit is there: the
        // loads are unconditional, so the compiler's count of outstanding
        // loads is exact and each wait leaves the other set in flight (the
        // two first items are loaded both here or both early: one set
        // loaded early and one here would leave the count inexact).
        const bool pre = early && b0 == 0;
        const int rb = row0 + b0;
        int a = __builtin_amdgcn_readfirstlane(wave), b = a + kWaves;  // uniform
        if (b < items) {
            if (!pre) {
                down_item_load(p, A, a, S, nc, base0, base1, rb, lane);
                down_item_load(p, B, b, S, nc, base0, base1, rb, lane);
            }
            for (;;) {
                const int n2 = next_local_pair(sh, lane);
                if (n2 >= items) break;
                down_item_finish(sh, A, act, nv, a, S, nc, lane);
                a = n2;
                down_item_load(p, A, a, S, nc, base0, base1, rb, lane);
                down_item_finish(sh, B, act, nv, b, S, nc, lane);
                b = n2 + 1;
                down_item_load(p, B, b, S, nc, base0, base1, rb, lane);
            }
            down_item_finish(sh, A, act, nv, a, S, nc, lane);
            down_item_finish(sh, B, act, nv, b, S, nc, lane);
        } else if (a < items) {
            if (!pre) down_item_load(p, A, a, S, nc, base0, base1, rb, lane);
            down_item_finish(sh, A, act, nv, a, S, nc, lane);
        }
        __syncthreads();
        // h = bf16(h + bf16(s_j * bf16(d_j))) for j = 0, 1 in order
        for (int r = tid; r < nb_rows; r += kThreads) {
            float d0 = 0.f, d1 = 0.f;
            for (int sg = 0; sg < S; ++sg) {
                d0 += sh.part[(r * 2 + 0) * kMaxSegments + sg];
                d1 += sh.part[(r * 2 + 1) * kMaxSegments + sg];
            }
            uint16_t *hp = p.hidden + row0 + b0 + r;
            float h = bf2f(known && b0 == 0 ? hpre : ld_dev16(hp));  // r == tid in the first batch
            h = rbf(h + rbf(s0 * rbf(d0)));
            h = rbf(h + rbf(s1 * rbf(d1)));
            st_dev16(hp, f2bf(h));
        }
        if (tid == 0) sh.next_item = 2 * kWaves;
        __syncthreads();
    }
    drain_and_sync();
    arrive(p, bar_at(p, layer, 6), 2 * (end - start));
    stamp(tim, MK_TEVENT_DONE_GMEM_STORE);
    return true;
}

// ---------------------------------------------------------------------------
// opcode 8: SpeculativeExpertPredict  (python_vm.py:356-371)
// ---------------------------------------------------------------------------

template <int kE>
__device__ __forceinline__ bool op_predict(kp_c &p, SharedState &sh, u32x4 *act, ins_t *ins, const Ctx &c,
                           int32_t *tim) {
    const int layer = __builtin_amdgcn_readfirstlane(ins[1]);
    if (layer < 0 || layer >= p.num_layers) {
        report_error(p, MK_ERR_BAD_INSTRUCTION, c, 8, layer, 0, 0);
        return false;
    }
    const uint16_t *weights = p.predictor != nullptr ? p.predictor : p.router;
    if (p.late_loads && layer > 0 && !wait_ge(p, sh, bar_at(p, layer - 1, 6), p.down_arrivals, c, 8, layer))
        return false;
    RouterRegs<kE> rr;
    router_prefetch<kE>(p, sh, layer, weights, rr);
    if (!p.late_loads && layer > 0) {
        stamp(tim, MK_TEVENT_AT_GMEM_WAIT);
        if (!wait_ge(p, sh, bar_at(p, layer - 1, 6), p.down_arrivals, c, 8, layer)) return false;
        stamp(tim, MK_TEVENT_DONE_GMEM_WAIT);
    }
    float logits[Experts<kE>::kMax];
    rms_router<kE>(p, sh, act, layer, weights, rr, tim, logits);
    const Top2 t = softmax_top2<kE>(p, logits);
    if (threadIdx.x == 0) {
        st_dev32(p.pred_idx, (uint32_t)t.i0);
        st_dev32(p.pred_idx + 1, (uint32_t)t.i1);
    }
    drain_and_sync();
    arrive(p, bar_at(p, layer, 8), 1);
    stamp(tim, MK_TEVENT_DONE_GMEM_STORE);
    return true;
}

// ---------------------------------------------------------------------------
// attention side and LM head: opcodes 1-4 and 7 (python_vm.py:61-222, 321-345)
// ---------------------------------------------------------------------------

__device__ __forceinline__ bool need_attention(kp_c &p, const Ctx &c, int op, int layer) {
    if (p.attn) return true;
    report_error(p, MK_ERR_UNSUPPORTED_OPCODE, c, op, layer, 0, op);
    return false;
}

// Wait until the counter each of the first n (<= 64) lanes of wave 0 points
// at reaches `expected`.  Every control value is wave-uniform (ballot,
// readfirstlane); the result is broadcast to the workgroup like wait_ge's.
__device__ __forceinline__ bool wait_lanes_ge(kp_c &p, SharedState &sh, const int32_t *mine, int n, int expected,
                              const Ctx &c, int opcode, int layer) {
    if (threadIdx.x < 64) {
        const int lane = threadIdx.x;
        int ok = 1, nap = 1;
        const uint64_t t0 = __builtin_amdgcn_s_memrealtime();
        for (;;) {
            int v = expected;
            if (lane < n) v = (int)ld_dev32(mine);
            const uint64_t shortfall = __ballot(v < expected);
            if (shortfall == 0) break;
            const int other = __builtin_amdgcn_readfirstlane(
                (int)__hip_atomic_load(p.status, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
            if (other != 0) {
                ok = 0;
                break;
            }
            if (__builtin_amdgcn_s_memrealtime() - t0 > (uint64_t)p.timeout_ticks) {
                if (lane == (int)__builtin_ctzll(shortfall)) report_error_lane(p, MK_ERR_TIMEOUT, c, opcode, layer, expected, v);
                ok = 0;
                break;
            }
            for (int i = 0; i < nap; ++i) __builtin_amdgcn_s_sleep(1);
            if (nap < p.spin_max) nap *= 2;
        }
        if (lane == 0) sh.flag = ok;
    }
    __syncthreads();
    const bool ok = sh.flag != 0;
    __syncthreads();
    return ok;
}

// act[0 .. H/8) = bf16(w * bf16(h * 1/sqrt(mean(h^2) + eps))) of the current
// hidden state (python_vm rms_norm, lat/python_vm.py:50-56).  Ends with a
// workgroup barrier.
__device__ __forceinline__ void rms_to_lds(kp_c &p, SharedState &sh, u32x4 *act, const uint16_t *w) {
    const int tid = threadIdx.x, nv = p.H >> 3;
    float ss = 0.f;
    for (int v = tid; v < nv; v += kThreads) ss += sumsq8(ld_dev128(p.hidden, (uint32_t)v * 16u));
    ss = block_sum(ss, sh.red_ss);
    const float r = 1.0f / sqrtf(ss / (float)p.H + p.eps);
    const u32x4 *w4 = reinterpret_cast<const u32x4 *>(w);
    for (int v = tid; v < nv; v += kThreads) act[v] = norm8(ld_dev128(p.hidden, (uint32_t)v * 16u), w4[v], r);
    __syncthreads();
}

// Rows [r0, r0 + nrows) (nrows even) of a row-major bf16 matrix with row
// stride `ld` (elements), columns [col0, col0 + nc * 512), dotted with the
// LDS vector x (8 bf16 per u32x4, starting at column col0); pairs of rows per
// wave item, claimed from the LDS counter (reset by the caller before a
// barrier).  fn(row, fp32 sum) is called by lane 0 of the wave.
template <typename Fn>
__device__ __forceinline__ void matvec_rows(SharedState &sh, const uint16_t *mat, size_t ld, int col0, int nc,
                                            const u32x4 *x, int r0, int nrows, Fn fn) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    for (int it = wave; 2 * it < nrows; it = next_local_item(sh, lane)) {
        const int ra = r0 + 2 * it;
        float aa = 0.f, ab = 0.f;
        dot_pair(mat + (size_t)ra * ld + col0, mat + (size_t)(ra + 1) * ld + col0, x, x, nc, lane, aa, ab);
        aa = wave_sum(aa);
        ab = wave_sum(ab);
        if (lane == 0) {
            fn(ra, aa);
            fn(ra + 1, ab);
        }
    }
}

// Row pairs kWaves .. kWaves + nst - 1 of a matvec_rows_ahead (rows r0 + 2 q
// and the next, nc chunks from column col0) streamed into LDS at `stage`
// with global_load_lds, each wave its pairs q = kWaves + wave (+ kWaves ..):
// pair q, row j, chunk c at stage[((2 (q - kWaves) + j) nc + c) 64], lane
// order.  They land before the workgroup's next barrier.
__device__ __forceinline__ void stage_pairs(const uint16_t *mat, size_t ld, int col0, int nc, int r0, int nst,
                                            u32x4 *stage) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    for (int q = wave; q < nst; q += kWaves) {
        const uint16_t *ra = mat + (size_t)(r0 + 2 * (q + kWaves)) * ld + col0;
        for (int j = 0; j < 2; ++j)
            for (int ch = 0; ch < nc; ++ch)
                __builtin_amdgcn_global_load_lds(
                    (global_void_t *)(reinterpret_cast<const u32x4 *>(ra + j * ld) + ch * 64 + lane),
                    (lds_void_t *)(stage + ((2 * q + j) * nc + ch) * 64), 16, 0, 0);
    }
}

// matvec_rows whose first item per wave was loaded by pair_ahead_load with
// the same arguments, except the row pairs sbase .. sbase + nst - 1, which
// were staged at `stage` (row-major 512-column chunks in lane order) by
// stage_pairs (sbase = kWaves) or stage_oproj_rows (sbase = 0: every pair,
// nothing loaded ahead).  The summation order is the same in all three
// forms.  fn(row, sum) per row, called by lane 0.
template <typename Fn>
__device__ __forceinline__ void matvec_rows_ahead(SharedState &sh, const PairAhead &pre, const uint16_t *mat,
                                                  size_t ld, int col0, int nc, const u32x4 *x, int r0, int nrows,
                                                  Fn fn, const u32x4 *stage = nullptr, int nst = 0,
                                                  int sbase = kWaves) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    auto staged_pair = [&](int q, float &aa, float &ab) {
        const u32x4 *sa = stage + (2 * q) * nc * 64 + lane, *sb = sa + nc * 64;
        for (int ch = 0; ch < nc; ++ch) {
            aa = dot8(sa[ch * 64], x[lane + ch * 64], aa);
            ab = dot8(sb[ch * 64], x[lane + ch * 64], ab);
        }
    };
    if (2 * wave < nrows) {
        const int ra = r0 + 2 * wave;
        float aa = 0.f, ab = 0.f;
        if (sbase == 0 && wave < nst) {
            staged_pair(wave, aa, ab);
        } else {
#pragma unroll
            for (int i = 0; i < kAheadChunks; ++i)
                if (i < nc) {
                    aa = dot8(pre.a[i], x[lane + i * 64], aa);
                    ab = dot8(pre.b[i], x[lane + i * 64], ab);
                }
            if (nc > kAheadChunks) {
                const uint16_t *row_a = mat + (size_t)ra * ld + col0 + kAheadChunks * kChunkElems;
                dot_pair(row_a, row_a + ld, x + kAheadChunks * 64, x + kAheadChunks * 64, nc - kAheadChunks, lane,
                         aa, ab);
            }
        }
        aa = wave_sum(aa);
        ab = wave_sum(ab);
        if (lane == 0) {
            fn(ra, aa);
            fn(ra + 1, ab);
        }
    }
    for (int it = next_local_item(sh, lane); 2 * it < nrows; it = next_local_item(sh, lane)) {
        const int ra = r0 + 2 * it;
        float aa = 0.f, ab = 0.f;
        if (it - sbase < nst)
            staged_pair(it - sbase, aa, ab);
        else
            dot_pair(mat + (size_t)ra * ld + col0, mat + (size_t)(ra + 1) * ld + col0, x, x, nc, lane, aa, ab);
        aa = wave_sum(aa);
        ab = wave_sum(ab);
        if (lane == 0) {
            fn(ra, aa);
            fn(ra + 1, ab);
        }
    }
}

// ---- opcode 1: Mixtral_QKV  (python_vm.py:61-118) -------------------------

__device__ __forceinline__ bool op_qkv(kp_c &p, SharedState &sh, u32x4 *act, ins_t *ins, const Ctx &c,
                       int32_t *tim) {
    const int layer = __builtin_amdgcn_readfirstlane(ins[1]);
    const int b0 = __builtin_amdgcn_readfirstlane(ins[2]);
    const int b1 = __builtin_amdgcn_readfirstlane(ins[3]);
    if (!need_attention(p, c, 1, layer)) return false;
    attn_c &a = attn_of(p);  // valid: attention tensors are present
    const int D = a.D, qkv_rows = (a.Hq + 2 * a.Hkv) * D;
    if (layer < 0 || layer >= p.num_layers || b0 < 0 || b1 < b0 || (int64_t)b1 * a.qkv_bs > qkv_rows) {
        report_error(p, MK_ERR_BAD_INSTRUCTION, c, 1, layer, b0, b1);
        return false;
    }
    if (threadIdx.x == 0) sh.next_item = kWaves;
    const int r0 = b0 * a.qkv_bs, nrows = (b1 - b0) * a.qkv_bs;
    const uint16_t *wq = a.qkv + (size_t)layer * qkv_rows * p.H;
    auto wait = [&] { return layer == 0 || wait_ge(p, sh, bar_at(p, layer - 1, 6), p.down_arrivals, c, 1, layer); };
    if (p.late_loads && !wait()) return false;
    PairAhead pre;
    stamp(tim, MK_TEVENT_FIRST_LOAD);
    const int nc = p.H / kChunkElems;
    pair_ahead_load(pre, wq, (size_t)p.H, 0, nc, r0, nrows);
    // the pairs after the ones loaded ahead go to LDS, after the normed
    // hidden state and the block's outputs, as far as the launch's LDS holds
    const int soff16 = (((p.H * 2 + nrows * 4) + 1023) / 1024) * 64;  // u32x4 units
    const int nst = min(max(nrows / 2 - kWaves, 0), max(p.lds_bytes / 16 - soff16, 0) / (2 * nc * 64));
    stage_pairs(wq, (size_t)p.H, 0, nc, r0, nst, act + soff16);
    stamp(tim, MK_TEVENT_AT_GMEM_WAIT);
    if (!p.late_loads && !wait()) return false;
    stamp(tim, MK_TEVENT_DONE_GMEM_WAIT);
    rms_to_lds(p, sh, act, a.attn_ln + (size_t)layer * p.H);

    float *rowv = reinterpret_cast<float *>(act + (p.H >> 3));  // the block's outputs, bf16-rounded
    matvec_rows_ahead(
        sh, pre, wq, (size_t)p.H, 0, nc, act, r0, nrows, [&](int r, float s) { rowv[r - r0] = rbf(s); },
        act + soff16, nst);
    __syncthreads();

    // RoPE on q and k rows (interleaved pairs (2i, 2i+1) share cos/sin[2i]):
    // y = x * cos + rot(x) * sin in fp32 without contraction, rot(a, b) =
    // (-b, a); then q -> q_post_rope, k/v -> the caches at pos_id.
    const int k0 = a.Hq * D, v0 = k0 + a.Hkv * D;
    const size_t kv_base = ((size_t)layer * a.T + p.pos) * (size_t)(a.Hkv * D);
    for (int i = threadIdx.x; i < nrows; i += kThreads) {
        const int r = r0 + i;
        float y = rowv[i];
        if (r < v0) {
            const int d = r % D;
            const float partner = rowv[i ^ 1];
            const float cs = a.rope_cos[(size_t)p.pos * D + d], sn = a.rope_sin[(size_t)p.pos * D + d];
            y = __fadd_rn(__fmul_rn(y, cs), __fmul_rn((d & 1) ? partner : -partner, sn));
        }
        const uint32_t bits = f2bf(y);
        if (r < k0)
            st_dev16(a.q_rope + r, bits);
        else if (r < v0)
            st_dev16(a.kc + kv_base + (r - k0), bits);
        else
            st_dev16(a.vc + kv_base + (r - v0), bits);
    }
    drain_and_sync();
    // one arrival per block on its head's counter
    const int bph = D / a.qkv_bs;
    for (int b = b0 + (int)threadIdx.x; b < b1; b += kThreads)
        __hip_atomic_fetch_add(bar_at(p, layer, 1) + b / bph, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    stamp(tim, MK_TEVENT_DONE_GMEM_STORE);
    return true;
}

// ---- opcode 2: Mixtral_PartialAttn  (python_vm.py:125-159) ----------------

// Sum over each group of G consecutive lanes (G = 8 or 16); every lane of a
// group ends with the group's sum.
__device__ __forceinline__ float group_sum(float v, int G) {
    v += dpp_add_src<0xb1>(v);   // quad_perm [1, 0, 3, 2]
    v += dpp_add_src<0x4e>(v);   // quad_perm [2, 3, 0, 1]
    v += dpp_add_src<0x141>(v);  // row_half_mirror: groups of 8
    if (G == 16) v += dpp_add_src<0x140>(v);  // row_mirror: groups of 16
    return v;
}

// The value lane l ^ o holds, for o in {8, 16, 32} (wave-uniform o): one
// VALU operation each instead of an LDS permute -- DPP row_ror:8 within a
// row of 16 lanes, and gfx950's v_permlane16_swap / v_permlane32_swap
// across rows (applied to a register and its copy, the second result holds,
// in the lanes below the swapped boundary, the partner rows' values).
__device__ __forceinline__ float lane_xor(float v, int o, int lane) {
    const uint32_t u = __float_as_uint(v);
    if (o == 32) {
        const auto r = __builtin_amdgcn_permlane32_swap(u, u, false, false);
        return __uint_as_float(lane < 32 ? r[1] : r[0]);
    }
    if (o == 16) {
        const auto r = __builtin_amdgcn_permlane16_swap(u, u, false, false);
        return __uint_as_float((lane & 16) == 0 ? r[1] : r[0]);
    }
    return __int_as_float(__builtin_amdgcn_update_dpp(0, (int)u, 0x128, 0xf, 0xf, false));  // row_ror:8
}

constexpr float kLog2e = 1.4426950408889634f;

// Scores are kept in log2 units: q is pre-scaled by attn_scale * log2(e), so
// that exp(s) = exp2(s2) and a partition's LSE is log2(sum exp2(s2 - M2)) + M2.
__device__ __forceinline__ float exp2_fast(float x) { return __builtin_amdgcn_exp2f(x); }

__device__ __forceinline__ void widen8(u32x4 x, float (&f)[8]) {
    const uint32_t w[4] = {x.x, x.y, x.z, x.w};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        f[2 * j] = bf2f(w[j] & 0xffffu);
        f[2 * j + 1] = __uint_as_float(w[j] & 0xffff0000u);
    }
}

// K/V staging for opcode 2: the partition's rows pass through an LDS ring of
// `kv_ring` chunks.  A chunk holds CT = 8 KiB / (2 D) positions: their K rows
// (8 KiB), then their V rows (8 KiB).  Wave w stages and reads only its own
// 1 KiB of each half (positions w * TPW .. + TPW of the chunk), one 16-byte
// piece (dims dp * 8 .. + 8 of position slot) per lane in lane order, which
// is the order global_load_lds writes LDS in; so staging and use need no
// workgroup barrier, only the wave's own wait for its loads.
constexpr int kKvChunkBytes = 16384;
constexpr int kKvRingMax = 8;
constexpr int kAttnSub = 4;  // ring slots scored per softmax rescale


__device__ __forceinline__ void stage_kv(unsigned char *dst, const uint16_t *kbase, const uint16_t *vbase,
                                         uint32_t row_bytes, int t, int dp) {
    const size_t off = (size_t)t * row_bytes + (size_t)dp * 16u;
    __builtin_amdgcn_global_load_lds((global_void_t *)(reinterpret_cast<const char *>(kbase) + off),
                                     (lds_void_t *)dst, 16, 0, 0);
    __builtin_amdgcn_global_load_lds((global_void_t *)(reinterpret_cast<const char *>(vbase) + off),
                                     (lds_void_t *)(dst + kKvChunkBytes / 2), 16, 0, 0);
}

// Split-KV partial attention of query heads kv * GQA .. + GQA over the
// partition's positions [t0, t1).  Positions before pos_id were written by
// earlier launches, so the first ring of them is staged before the wait on
// the QKV counters; the new position's rows (written by this launch) are
// read after it with device-coherent loads and patched into the ring.
// Scores are kept in log2 units (q pre-scaled by attn_scale * log2(e)), so
// exp(s) = exp2(s2) and the partition's LSE is log2(L) + M.
template <int GQA>
__device__ __forceinline__ bool partial_attn(kp_c &p, attn_c &a, SharedState &sh, u32x4 *act, const Ctx &c,
                             int layer, int kv, int nparts, int pidx, int32_t *tim) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int D = a.D, G = D / 8, TPW = 64 / G, CT = kWaves * TPW;
    const int slot = lane / G, dp = lane % G;
    const int h0 = kv * GQA;
    const int nb = a.kv_ring;
    const int pos = (int)p.pos, seq = pos + 1;
    const int total = (seq + a.kv_bs - 1) / a.kv_bs;
    const int per = (total + nparts - 1) / nparts;
    const int tb0 = pidx * per, tb1 = min(tb0 + per, total);
    const int t0 = tb0 * a.kv_bs, t1 = min(tb1 * a.kv_bs, seq);
    const int nch = t1 > t0 ? (t1 - t0 + CT - 1) / CT : 0;
    const int first = t0 + wave * TPW + slot;  // this lane's position in chunk 0
    const int wpos = t0 + __builtin_amdgcn_readfirstlane(wave) * TPW;  // the wave's first position in chunk 0
    const bool has_new = pos >= t0 && pos < t1;
    const int c_new = has_new ? (pos - t0) / CT : -1;
    const bool own_new = has_new && ((pos - t0) % CT) / TPW == wave;  // uniform

    unsigned char *ring = reinterpret_cast<unsigned char *>(act);
    unsigned char *wave_lds = ring + wave * 1024;  // the wave's piece of ring slot 0
    u32x4 *kl = reinterpret_cast<u32x4 *>(wave_lds) + lane;
    // K and V of this layer and KV head: position t at byte (t * Hkv * D) * 2
    const uint16_t *kbase = a.kc + (size_t)layer * a.T * a.Hkv * D + (size_t)kv * D;
    const uint16_t *vbase = a.vc + (size_t)layer * a.T * a.Hkv * D + (size_t)kv * D;
    const uint32_t row_bytes = (uint32_t)(a.Hkv * D * 2);
    // Chunk ch lives in ring slot ch % nb.  Groups of kAttnSub chunks are
    // computed in order; with an 8-chunk ring two groups are resident, and
    // a consumed group's slots are restaged with the group two later while
    // the next group is computed.
    auto stage_chunks = [&](int c0, int c1) {
        for (int ch = c0; ch < c1 && ch < nch; ++ch) {
            const int t = first + ch * CT;
            stage_kv(wave_lds + (ch % nb) * kKvChunkBytes, kbase, vbase, row_bytes, (t < t1 && t != pos) ? t : t0,
                     dp);
        }
    };
    // producers: the GQA query heads, the key head and the value head
    const int bph = D / a.qkv_bs;
    const int32_t *bar_qkv = bar_at(p, layer, 1);
    const int32_t *mine = bar_qkv + (lane < GQA ? h0 + lane : lane == GQA ? a.Hq + kv : a.Hq + a.Hkv + kv);
    if (p.late_loads && !wait_lanes_ge(p, sh, mine, GQA + 2, bph, c, 2, layer)) return false;
    stamp(tim, MK_TEVENT_FIRST_LOAD);
    stage_chunks(0, nb);
    stamp(tim, MK_TEVENT_AT_GMEM_WAIT);
    if (!p.late_loads && !wait_lanes_ge(p, sh, mine, GQA + 2, bph, c, 2, layer)) return false;
    stamp(tim, MK_TEVENT_DONE_GMEM_WAIT);

    const float qscale = a.attn_scale * kLog2e;
    float q[GQA][8];
#pragma unroll
    for (int h = 0; h < GQA; ++h) {
        widen8(ld_dev128(a.q_rope, (uint32_t)(((h0 + h) * D + dp * 8) * 2)), q[h]);
#pragma unroll
        for (int j = 0; j < 8; ++j) q[h][j] *= qscale;
    }
    // the new position's rows, device-coherent: loaded now, patched over the
    // row t0 staged in their place once their chunk has landed
    u32x4 kn = {0u, 0u, 0u, 0u}, vn = {0u, 0u, 0u, 0u};
    if (own_new) {
        const uint32_t off = (uint32_t)pos * row_bytes + (uint32_t)dp * 16u;
        kn = ld_dev128(kbase, off);
        vn = ld_dev128(vbase, off);
    }
    float M[GQA], L[GQA], acc[GQA][8];
#pragma unroll
    for (int h = 0; h < GQA; ++h) {
        M[h] = -INFINITY;
        L[h] = 0.f;
#pragma unroll
        for (int j = 0; j < 8; ++j) acc[h][j] = 0.f;
    }
    const bool two = nb >= 2 * kAttnSub;  // two groups resident (uniform)
    const int ngroups = (nch + kAttnSub - 1) / kAttnSub;
    for (int g = 0; g < ngroups; ++g) {
        const int cg = g * kAttnSub;
        if (g == 0) {
            __builtin_amdgcn_s_waitcnt(0);  // the first ring (and the new rows) landed
            stamp(tim, MK_TEVENT_FIRST_USE);
        } else if (two) {
            // everything but the next group's loads (2 per chunk) has landed
            const int next = min(max(nch - cg - kAttnSub, 0), kAttnSub);
            switch (next) {
            case 0: asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); break;
            case 1: asm volatile("s_waitcnt vmcnt(2)" ::: "memory"); break;
            case 2: asm volatile("s_waitcnt vmcnt(4)" ::: "memory"); break;
            case 3: asm volatile("s_waitcnt vmcnt(6)" ::: "memory"); break;
            default: asm volatile("s_waitcnt vmcnt(8)" ::: "memory"); break;
            }
        } else {
            __builtin_amdgcn_s_waitcnt(0);
        }
        if (own_new && c_new >= cg && c_new < cg + kAttnSub && first + c_new * CT == pos) {
            kl[(c_new % nb) * (kKvChunkBytes / 16)] = kn;
            kl[(c_new % nb) * (kKvChunkBytes / 16) + kKvChunkBytes / 32] = vn;
        }
        // scores of the group's chunks
        float sc[GQA][kAttnSub];
#pragma unroll
        for (int u = 0; u < kAttnSub; ++u) {
            const int ch = cg + u, k = ch % nb;
            // chunks where every position of this wave is past the
            // partition (the last one, partly filled) are skipped: their
            // scores are -inf and their terms zero (uniform per wave)
            const bool live = ch < nch && wpos + ch * CT < t1;
            const bool valid = live && first + ch * CT < t1;
            float kf[8];
            if (live) widen8(kl[k * (kKvChunkBytes / 16)], kf);
#pragma unroll
            for (int h = 0; h < GQA; ++h) {
                float d = 0.f;
                if (live) {
#pragma unroll
                    for (int j = 0; j < 8; ++j) d = fmaf(q[h][j], kf[j], d);
                    d = group_sum(d, G);
                }
                sc[h][u] = valid ? d : -INFINITY;
            }
        }
        // rescale the slot's running state once, to the new max
        float ref[GQA];
#pragma unroll
        for (int h = 0; h < GQA; ++h) {
            float mb = M[h];
#pragma unroll
            for (int u = 0; u < kAttnSub; ++u) mb = fmaxf(mb, sc[h][u]);
            ref[h] = mb == -INFINITY ? 0.f : mb;
            const float alpha = exp2_fast(M[h] - ref[h]);  // 0 while M is -inf, 1 if the max holds
            L[h] *= alpha;
#pragma unroll
            for (int j = 0; j < 8; ++j) acc[h][j] *= alpha;
            M[h] = mb;
        }
#pragma unroll
        for (int u = 0; u < kAttnSub; ++u) {
            const int ch = cg + u, k = ch % nb;
            if (ch >= nch || wpos + ch * CT >= t1) continue;  // uniform per wave, as above
            // rows staged for masked positions may hold anything
            // (the row pos_id is read before this launch writes it)
            const u32x4 vraw = first + ch * CT < t1 ? kl[k * (kKvChunkBytes / 16) + kKvChunkBytes / 32]
                                                    : u32x4{0u, 0u, 0u, 0u};
            float vf[8];
            widen8(vraw, vf);
#pragma unroll
            for (int h = 0; h < GQA; ++h) {
                const float pr = exp2_fast(sc[h][u] - ref[h]);  // 0 for masked positions
                L[h] += pr;
#pragma unroll
                for (int j = 0; j < 8; ++j) acc[h][j] = fmaf(pr, vf[j], acc[h][j]);
            }
        }
        // this group's slots are free (its LDS reads fed the sums above):
        // restage them with the group that maps onto them
        const int cn = cg + (two ? 2 : 1) * kAttnSub;
        if (cn < nch) stage_chunks(cn, cn + kAttnSub);
    }

    stamp(tim, MK_TEVENT_AT_GMEM_STORE);  // wave 0's positions done
    // fold the token slots of the wave (lanes with the same dp) to the wave max
    const bool packed = G == 16;  // uniform: head dim 128, four slots = the wave's four rows of 16 lanes
#pragma unroll
    for (int h = 0; h < GQA; ++h) {
        // partners at lane distance 8 (head dim 64 only), 16 and 32
        float mw = M[h];
        if (G == 8) mw = fmaxf(mw, lane_xor(mw, 8, lane));
        mw = fmaxf(mw, lane_xor(mw, 16, lane));
        mw = fmaxf(mw, lane_xor(mw, 32, lane));
        const float f = M[h] == -INFINITY ? 0.f : exp2_fast(M[h] - mw);
        L[h] *= f;
#pragma unroll
        for (int j = 0; j < 8; ++j) acc[h][j] *= f;
#pragma unroll
        for (int k = 0; k < 3; ++k) {
            const int o = 8 << k;
            if (o < G) continue;
            L[h] += lane_xor(L[h], o, lane);
            if (!packed) {
#pragma unroll
                for (int j = 0; j < 8; ++j) acc[h][j] += lane_xor(acc[h][j], o, lane);
            }
        }
        M[h] = mw;
    }
    // per-wave partials to LDS after the ring: m, l [kWaves][GQA], acc [kWaves][GQA][D]
    float *wm = reinterpret_cast<float *>(ring + (size_t)nb * kKvChunkBytes);
    float *wl = wm + kWaves * GQA;
    float *wacc = wl + kWaves * GQA;
    if (lane == 0) {
#pragma unroll
        for (int h = 0; h < GQA; ++h) {
            wm[wave * GQA + h] = M[h];
            wl[wave * GQA + h] = L[h];
        }
    }
    if (packed) {
        // The four rows' acc summed two registers per swap: v_permlane32_swap
        // of (a_j, a_{j+4}) plus an add leaves a_j in the lower half and
        // a_{j+4} in the upper (rows 0+2 and 1+3 added); v_permlane16_swap of
        // (s_j, s_{j+2}) plus an add leaves in row r the whole sum of a_{j+2r}.
        // Row r of t0, t1 then holds dims dp * 8 + 2r, + 1: every lane
        // stores two.  Six swaps per head where lane exchanges take sixteen.
#pragma unroll
        for (int h = 0; h < GQA; ++h) {
            float s[4];
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(acc[h][j]),
                                                                __float_as_uint(acc[h][j + 4]), false, false);
                s[j] = __uint_as_float(r[0]) + __uint_as_float(r[1]);
            }
            float t[2];
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(s[j]), __float_as_uint(s[j + 2]),
                                                                false, false);
                t[j] = __uint_as_float(r[0]) + __uint_as_float(r[1]);
            }
            *reinterpret_cast<float2 *>(wacc + (wave * GQA + h) * D + dp * 8 + 2 * slot) = make_float2(t[0], t[1]);
        }
    } else if (slot == 0) {
#pragma unroll
        for (int h = 0; h < GQA; ++h)
#pragma unroll
            for (int j = 0; j < 8; ++j) wacc[(wave * GQA + h) * D + dp * 8 + j] = acc[h][j];
    }
    __syncthreads();
    stamp(tim, 55);  // every wave's partials are in LDS
    for (int i = threadIdx.x; i < GQA * D; i += kThreads) {
        const int h = i / D, d = i % D;
        float Mx = -INFINITY;
        for (int w = 0; w < kWaves; ++w) Mx = fmaxf(Mx, wm[w * GQA + h]);
        float Ls = 0.f, O = 0.f;
        if (Mx != -INFINITY) {
            for (int w = 0; w < kWaves; ++w) {
                const float mw = wm[w * GQA + h];
                if (mw == -INFINITY) continue;
                const float f = exp2_fast(mw - Mx);
                Ls += wl[w * GQA + h] * f;
                O += wacc[(w * GQA + h) * D + d] * f;
            }
        }
        const float out = Ls > 0.f ? O / Ls : 0.f;
        if (a.skip_red) {
            st_dev16(a.attn_out + (h0 + h) * D + d, f2bf(out));
        } else {
            st_dev32(a.out_int + ((size_t)(h0 + h) * a.P + pidx) * D + d, __float_as_uint(out));
            if (d == 0) {
                const float lse = Ls > 0.f ? log2f(Ls) + Mx : -INFINITY;
                st_dev32(a.lse_int + (size_t)(h0 + h) * a.P + pidx, __float_as_uint(lse));
            }
        }
    }
    stamp(tim, 56);  // thread 0's merged outputs stored
    drain_and_sync();
    if (a.skip_red)
        arrive(p, bar_at(p, layer, 3), GQA);
    else if (threadIdx.x < GQA)
        __hip_atomic_fetch_add(bar_at(p, layer, 2) + h0 + threadIdx.x, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    stamp(tim, MK_TEVENT_DONE_GMEM_STORE);
    return true;
}

__device__ __forceinline__ bool op_partial_attn(kp_c &p, SharedState &sh, u32x4 *act, ins_t *ins, const Ctx &c,
                                int32_t *tim) {
    const int layer = __builtin_amdgcn_readfirstlane(ins[1]);
    const int kv = __builtin_amdgcn_readfirstlane(ins[2]);
    const int nparts = __builtin_amdgcn_readfirstlane(ins[3]);
    const int pidx = __builtin_amdgcn_readfirstlane(ins[4]);
    if (!need_attention(p, c, 2, layer)) return false;
    attn_c &a = attn_of(p);  // valid: attention tensors are present
    if (layer < 0 || layer >= p.num_layers || kv < 0 || kv >= a.Hkv || nparts < 1 || pidx < 0 || pidx >= nparts ||
        (!a.skip_red && pidx >= a.P)) {
        report_error(p, MK_ERR_BAD_INSTRUCTION, c, 2, layer, kv, pidx);
        return false;
    }
    switch (a.Hq / a.Hkv) {
    case 1: return partial_attn<1>(p, a, sh, act, c, layer, kv, nparts, pidx, tim);
    case 2: return partial_attn<2>(p, a, sh, act, c, layer, kv, nparts, pidx, tim);
    case 3: return partial_attn<3>(p, a, sh, act, c, layer, kv, nparts, pidx, tim);
    default: return partial_attn<4>(p, a, sh, act, c, layer, kv, nparts, pidx, tim);
    }
}

// ---- opcode 3: Mixtral_AttnReduction  (python_vm.py:166-189) --------------

// The worker's next instruction `nx` (queue slot `slot`), when it is the
// O projection of `layer`: its weight rows depend on nothing, so opcode 3
// streams them into LDS (row-major 512-column chunks in lane order, at the
// staging offset) with global_load_lds while it waits for the partials,
// on waves 1.. (wave 0 polls).  A reduction worker otherwise starts its O
// projection's loads only when the reduction is done, and every other
// workgroup's opcode 5 then waits for it.
__device__ __forceinline__ void stage_oproj_rows(kp_c &p, const attn_c &a, SharedState &sh, u32x4 *act,
                                                 ins_t *nx, int slot, int layer) {
    if (p.late_loads || slot >= p.queue_len) return;
    const int op = __builtin_amdgcn_readfirstlane(nx[0]);
    const int l = __builtin_amdgcn_readfirstlane(nx[1]);
    const int b0 = __builtin_amdgcn_readfirstlane(nx[2]);
    const int b1 = __builtin_amdgcn_readfirstlane(nx[3]);
    const int red = __builtin_amdgcn_readfirstlane(nx[4]);
    if (op != 4 || l != layer || b0 < 0 || b1 <= b0 || (int64_t)b1 * p.oproj_bs > p.H || red != 0) return;
    const int K = a.Hq * a.D, nc = K / kChunkElems, nrows = (b1 - b0) * p.oproj_bs;
    if ((int64_t)p.stage_off16 * 16 + (int64_t)nrows * K * 2 > (int64_t)p.lds_bytes) return;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    if (wave >= 1) {
        const u32x4 *src = reinterpret_cast<const u32x4 *>(a.oproj + ((size_t)layer * p.H + (size_t)b0 * p.oproj_bs) * K) +
                           (threadIdx.x & 63);
        u32x4 *dst = act + p.stage_off16;
        const int n = nrows * nc;
        for (int pc = wave - 1; pc < n; pc += kWaves - 1)
            __builtin_amdgcn_global_load_lds((global_void_t *)(src + pc * 64), (lds_void_t *)(dst + pc * 64), 16, 0, 0);
    }
    if (threadIdx.x == 0) sh.ostage_slot = slot;
}

__device__ __forceinline__ bool op_attn_reduction(kp_c &p, SharedState &sh, u32x4 *act, ins_t *ins, const Ctx &c,
                                  int32_t *tim) {
    const int layer = __builtin_amdgcn_readfirstlane(ins[1]);
    const int hs = __builtin_amdgcn_readfirstlane(ins[2]);
    const int nparts = __builtin_amdgcn_readfirstlane(ins[3]);
    const int terminal = __builtin_amdgcn_readfirstlane(ins[4]);
    const int n = __builtin_amdgcn_readfirstlane(ins[5]);
    if (!need_attention(p, c, 3, layer)) return false;
    attn_c &a = attn_of(p);  // valid: attention tensors are present
    const int gqa = a.Hq / a.Hkv;
    // n < 0: the list is the range of partial slots 0 .. -n - 1, for more
    // partials than a 32-word instruction can list (no reference
    // counterpart: its lists stop at 25, demos/mixtral/mixtral.cuh)
    const bool range = n < 0;
    const int cnt = range ? -n : n;
    const int out_slot = range ? __builtin_amdgcn_readfirstlane(ins[6])
                         : n <= MK_INTS_PER_INSTRUCTION - 7 ? __builtin_amdgcn_readfirstlane(ins[6 + n])
                                                            : -1;
    bool bad = layer < 0 || layer >= p.num_layers || hs < 0 || hs + gqa > a.Hq || cnt < 1 ||
               (range ? cnt > 64 || cnt > a.P : n > MK_INTS_PER_INSTRUCTION - 7) ||
               (!terminal && (out_slot < 0 || out_slot >= a.P));
    for (int i = 0; !bad && !range && i < n; ++i) {
        const int s = ins[6 + i];
        bad = s < 0 || s >= a.P;
    }
    if (bad) {
        report_error(p, MK_ERR_BAD_INSTRUCTION, c, 3, layer, hs, n);
        return false;
    }
    if (MK_OSTAGE && p.ostage) stage_oproj_rows(p, a, sh, act, ins + MK_INTS_PER_INSTRUCTION, c.slot + 1, layer);
    stamp(tim, MK_TEVENT_AT_GMEM_WAIT);
    if (!wait_ge(p, sh, bar_at(p, layer, 2) + hs, nparts, c, 3, layer)) return false;
    stamp(tim, MK_TEVENT_DONE_GMEM_WAIT);
    const int D = a.D;
    // weights 2^(lse_k - max lse) and their sum: wave h, lane k (all n loads
    // in flight at once)
    static_assert(kRowBatchLds * 2 * kMaxSegments >= 4 * 64 + 4 + 64, "reduction staging fits in sh.part");
    float *wts = reinterpret_cast<float *>(sh.part);  // [gqa][64]
    float *den = wts + 4 * 64;                        // [gqa]
    int *slots = reinterpret_cast<int *>(den + 4);    // [cnt]
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    if (wave < gqa) {
        const int s = lane < cnt ? (range ? lane : ins[6 + lane]) : 0;
        float lse = lane < cnt ? __uint_as_float(ld_dev32(a.lse_int + (size_t)(hs + wave) * a.P + s)) : -INFINITY;
        float mx = lse;
        for (int o = 32; o >= 1; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o));
        const float f = lane < cnt ? exp2f(lse - mx) : 0.f;
        const float tot = wave_sum(f);
        wts[wave * 64 + lane] = f;
        if (lane == 0) den[wave] = tot;
        if (wave == 0 && lane < cnt) slots[lane] = s;
    }
    __syncthreads();
    stamp(tim, 52);  // the weights are in LDS
    // Four threads per (head, 4 dims): thread sub takes the partials sub,
    // sub + 4, ... with 16-byte loads (at most 16 in flight, all issued
    // before the first is used), then the quad adds its four sums
    // (quad_perm DPP) and its first thread stores the 4 outputs.
    const int ng = gqa * (D >> 2);
    for (int t = threadIdx.x; t < 4 * ng; t += kThreads) {  // whole quads: 4 * ng is a multiple of 4
        const int g = t >> 2, sub = t & 3;
        const int hl = g / (D >> 2), h = hs + hl, d = (g % (D >> 2)) * 4;
        const float *f = wts + hl * 64;
        u32x4 v[16];
#pragma unroll
        for (int u = 0; u < 16; ++u) {
            const int kk = sub + 4 * u;
            if (kk < cnt) {
                const int s = range ? kk : slots[kk];
                v[u] = ld_dev128(a.out_int, (uint32_t)(((h * a.P + s) * D + d) * 4));
            }
        }
        float num[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int u = 0; u < 16; ++u) {
            const int kk = sub + 4 * u;
            if (kk < cnt) {
                const float w = f[kk];
                num[0] = fmaf(__uint_as_float(v[u].x), w, num[0]);
                num[1] = fmaf(__uint_as_float(v[u].y), w, num[1]);
                num[2] = fmaf(__uint_as_float(v[u].z), w, num[2]);
                num[3] = fmaf(__uint_as_float(v[u].w), w, num[3]);
            }
        }
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            num[j] += dpp_add_src<0xb1>(num[j]);  // quad_perm [1, 0, 3, 2]
            num[j] += dpp_add_src<0x4e>(num[j]);  // quad_perm [2, 3, 0, 1]
        }
        if (sub == 0) {
            const float dn = den[hl];
            if (terminal) {
#pragma unroll
                for (int j = 0; j < 4; ++j) st_dev16(a.attn_out + h * D + d + j, f2bf(num[j] / dn));
            } else {
#pragma unroll
                for (int j = 0; j < 4; ++j)
                    st_dev32(a.out_int + ((size_t)h * a.P + out_slot) * D + d + j, __float_as_uint(num[j] / dn));
                if (d == 0) st_dev32(a.lse_int + (size_t)h * a.P + out_slot, __float_as_uint(logf(den[hl])));
            }
        }
    }
    stamp(tim, 53);  // thread 0's sums done and stored
    drain_and_sync();
    arrive(p, bar_at(p, layer, 3), gqa);
    stamp(tim, MK_TEVENT_DONE_GMEM_STORE);
    return true;
}

// ---- opcode 4: Mixtral_OProj  (python_vm.py:196-215) ----------------------

// Dense VM: the first items (gate and up rows, in item order) of an
// opcode-5 instruction `nx` of `layer` (queue slot `slot`) -- weights that
// depend on nothing -- streamed into LDS with global_load_lds while the
// workgroup waits anyway: by opcode 4 for its next instruction while it
// waits for the attention reduction, else by opcode 5 itself before its own
// wait.  Opcode 5 then starts on them the moment its wait ends.  Layout:
// item i, matrix j (0 gate, 1 up), chunk c is the 1 KiB at u32x4 index
// stage_off16 + ((2 i + j) nc + c) 64, lane order; item i is staged by wave
// i mod kWaves, which is also the wave that computes it.  The loads
// complete before the workgroup passes its next barrier.  Returns the items
// staged (uniform).  `publish` (opcode 4, for the next instruction) records
// them in sh.stage_slot / sh.stage_n for opcode 5 to find; opcode 5 staging
// its own items uses the return value, since its waves read sh.stage_slot
// at their own pace and a wave that saw it change would skip the staging
// and fall one workgroup barrier out of step with the others.
__device__ __forceinline__ int stage_dense_upgate(kp_c &p, SharedState &sh, u32x4 *act, ins_t *nx, int slot,
                                                  int layer, bool publish) {
    if (p.stage_items <= 0 || slot >= p.queue_len) return 0;
    const int op = __builtin_amdgcn_readfirstlane(nx[0]);
    const int l = __builtin_amdgcn_readfirstlane(nx[1]);
    const int n = __builtin_amdgcn_readfirstlane(nx[2]);
    if (op != 5 || l != layer || n < 1 || n > MK_INTS_PER_INSTRUCTION - 3) return 0;
    const int S = min(p.stage_items, n * p.expert_bs);
    const int nblocks = p.F / p.expert_bs;
    for (int k = 0; k * p.expert_bs < S; ++k) {
        const int b = __builtin_amdgcn_readfirstlane(nx[3 + k]);
        if (b < 0 || b >= nblocks) return 0;  // opcode 5 reports it
    }
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int nc = p.H / kChunkElems;
    for (int it = wave; it < S; it += kWaves) {
        const int k = it / p.expert_bs;
        const int row = __builtin_amdgcn_readfirstlane(nx[3 + k]) * p.expert_bs + it - k * p.expert_bs;
        const size_t off = ((size_t)layer * p.F + row) * (size_t)p.H;
        const u32x4 *wg = reinterpret_cast<const u32x4 *>(p.gate + off) + lane;
        const u32x4 *wu = reinterpret_cast<const u32x4 *>(p.up + off) + lane;
        for (int ch = 0; ch < nc; ++ch) {
            __builtin_amdgcn_global_load_lds((global_void_t *)(wg + ch * 64),
                                             (lds_void_t *)(act + p.stage_off16 + ((2 * it) * nc + ch) * 64), 16, 0, 0);
            __builtin_amdgcn_global_load_lds((global_void_t *)(wu + ch * 64),
                                             (lds_void_t *)(act + p.stage_off16 + ((2 * it + 1) * nc + ch) * 64), 16,
                                             0, 0);
        }
    }
    if (publish && threadIdx.x == 0) {
        sh.stage_slot = slot;
        sh.stage_n = S;
    }
    return S;
}

// Mixtral whole-model launches: the first items (a gate row and an up row
// each) of the opcode-5 instruction `nx` that follows this O projection in
// the queue (slot `slot`), of the expert opcode 8 predicted first, streamed
// into LDS by waves 1 .. stage_items (one item each, item w = wave w's first
// item there) with global_load_lds while the workgroup waits for the
// attention reduction -- the reference's speculative expert prefetch
// (mx/rms_router_matvec.cu:259-290), placed where HBM is idle: during
// partial attention and the reduction.  Only when the prediction is in and
// no reduction has arrived yet, so the loads land well before the wait
// ends (the O projection's later loads queue behind them).  Opcode 5 uses
// the rows if its routing picks the predicted expert first.  Wave 0 stages
// nothing: its thread 0 polls the counter.
__device__ __forceinline__ void stage_moe_upgate(kp_c &p, SharedState &sh, u32x4 *act, ins_t *nx, int slot,
                                                 int layer) {
    if (p.stage_items <= 0 || slot >= p.queue_len) return;
    const int op = __builtin_amdgcn_readfirstlane(nx[0]);
    const int l = __builtin_amdgcn_readfirstlane(nx[1]);
    const int start = __builtin_amdgcn_readfirstlane(nx[2]);
    const int nb = __builtin_amdgcn_readfirstlane(nx[3]);
    if (op != 5 || l != layer || start < 0 || nb < 1 || (int64_t)(start + nb) * p.expert_bs > p.F) return;
    if (threadIdx.x == 0) {
        // prediction counter, reduction counter and the prediction, one round trip
        const int32_t *pc = bar_at(p, layer, 8), *rc = bar_at(p, layer, 3);
        const int pv = counter_value(p, pc, spread_row(p, pc)), rv = counter_value(p, rc, spread_row(p, rc));
        const int e0 = (int)ld_dev32(p.pred_idx);
        sh.spec_e[0] = pv >= 1 && rv == 0 && e0 >= 0 && e0 < p.E ? e0 : -1;
    }
    __syncthreads();
    const int pe0 = __builtin_amdgcn_readfirstlane(sh.spec_e[0]);
    if (pe0 < 0) return;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int row0 = start * p.expert_bs, S = min(p.stage_items, nb * p.expert_bs - 1);
    if (wave >= 1 && wave <= S) {
        const int nc = p.H / kChunkElems;
        const size_t off = ((size_t)(layer * p.E + pe0) * p.F + row0 + wave) * (size_t)p.H;
        const u32x4 *wg = reinterpret_cast<const u32x4 *>(p.gate + off) + lane;
        const u32x4 *wu = reinterpret_cast<const u32x4 *>(p.up + off) + lane;
        u32x4 *dst = act + p.stage_off16 + (wave - 1) * 2 * nc * 64;
        for (int i = 0; i < nc; ++i) {
            __builtin_amdgcn_global_load_lds((global_void_t *)(wg + i * 64), (lds_void_t *)(dst + i * 64), 16, 0, 0);
            __builtin_amdgcn_global_load_lds((global_void_t *)(wu + i * 64), (lds_void_t *)(dst + (nc + i) * 64), 16,
                                             0, 0);
        }
    }
    if (threadIdx.x == 0) {
        sh.stage_slot = slot;
        sh.stage_n = S;
    }
}

__device__ __forceinline__ bool op_oproj(kp_c &p, SharedState &sh, u32x4 *act, ins_t *ins, const Ctx &c,
                         int32_t *tim) {
    const int layer = __builtin_amdgcn_readfirstlane(ins[1]);
    const int b0 = __builtin_amdgcn_readfirstlane(ins[2]);
    const int b1 = __builtin_amdgcn_readfirstlane(ins[3]);
    const int red = __builtin_amdgcn_readfirstlane(ins[4]);
    if (!need_attention(p, c, 4, layer)) return false;
    attn_c &a = attn_of(p);  // valid: attention tensors are present
    if (layer < 0 || layer >= p.num_layers || b0 < 0 || b1 < b0 || (int64_t)b1 * p.oproj_bs > p.H || red != 0) {
        report_error(p, MK_ERR_BAD_INSTRUCTION, c, 4, layer, b0, b1);
        return false;
    }
    if (threadIdx.x == 0) sh.next_item = kWaves;
    const int K = a.Hq * a.D;  // reduction length
    const uint16_t *wo = a.oproj + (size_t)layer * p.H * K;
    const int r0 = b0 * p.oproj_bs, nrows = (b1 - b0) * p.oproj_bs;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    // The residual rows of each wave's first item are final once the
    // previous layer's down-projection is complete (or at layer 0): read
    // them now instead of after the sums (one dependent load less).
    if (p.late_loads && !wait_ge(p, sh, bar_at(p, layer, 3), a.Hq, c, 4, layer)) return false;
    const bool hfinal = !p.late_loads &&
                        (layer == 0 || counter_reached(p, sh, bar_at(p, layer - 1, 6), p.down_arrivals)) &&
                        2 * wave < nrows;  // uniform
    const int rpre = r0 + 2 * wave;
    uint32_t hpair = 0;
    if (hfinal && lane == 0) hpair = ld_dev32(p.hidden + rpre);
    PairAhead pre;
    stamp(tim, MK_TEVENT_FIRST_LOAD);
    // rows staged in LDS by the preceding opcode 3 (stage_oproj_rows; its
    // loads were waited for before its last workgroup barrier): nothing to
    // load, and the staging area is taken
    const bool ostaged = MK_OSTAGE && __builtin_amdgcn_readfirstlane(sh.ostage_slot) == c.slot;
    if (!ostaged) {
        pair_ahead_load(pre, wo, (size_t)K, 0, K / kChunkElems, r0, nrows);
        if (p.E == 1)
            (void)stage_dense_upgate(p, sh, act, ins + MK_INTS_PER_INSTRUCTION, c.slot + 1, layer, true);
        else
            stage_moe_upgate(p, sh, act, ins + MK_INTS_PER_INSTRUCTION, c.slot + 1, layer);
    }
    stamp(tim, MK_TEVENT_AT_GMEM_WAIT);
    if (!p.late_loads && !wait_ge(p, sh, bar_at(p, layer, 3), a.Hq, c, 4, layer)) return false;
    stamp(tim, MK_TEVENT_DONE_GMEM_WAIT);
    for (int v = threadIdx.x; v < (K >> 3); v += kThreads) act[v] = ld_dev128(a.attn_out, (uint32_t)v * 16u);
    __syncthreads();
    auto add_row = [&](int r, float s) {
        uint16_t *hp = p.hidden + r;
        const uint32_t h = hfinal && r == rpre       ? (hpair & 0xffffu)
                           : hfinal && r == rpre + 1 ? (hpair >> 16)
                                                     : ld_dev16(hp);
        st_dev16(hp, f2bf(bf2f(h) + rbf(s)));
    };
    matvec_rows_ahead(sh, pre, wo, (size_t)K, 0, K / kChunkElems, act, r0, nrows, add_row, act + p.stage_off16,
                      ostaged ? nrows / 2 : 0, 0);
    drain_and_sync();
    if (ostaged && threadIdx.x == 0) sh.ostage_slot = -1;  // every thread has read it
    arrive(p, bar_at(p, layer, 4), b1 - b0);
    stamp(tim, MK_TEVENT_DONE_GMEM_STORE);
    return true;
}

// ---- LM-head row items ------------------------------------------------------

// Rows [row, row + nv) (nv <= NR) x NC chunks of 512 columns from col0 into
// registers, 16 B per lane per chunk.
template <int NR, int NC>
__device__ __forceinline__ void load_rows_upto(u32x4 (&w)[NR][NC], const uint16_t *mat, size_t ld, int row, int nv,
                                               int col0, int lane) {
#pragma unroll
    for (int i = 0; i < NR; ++i)
        if (i < nv) {
#pragma unroll
            for (int c = 0; c < NC; ++c)
                w[i][c] = load_stream(reinterpret_cast<const u32x4 *>(mat + (size_t)(row + i) * ld + col0) + c * 64 +
                                      lane);
        }
}

// Matvec of rows [r0, r0 + nrows) (an even count) over NC chunks from col0
// with the LDS vector x, in items of NR rows (NR * NC loads per lane in
// flight; a row pair of 512-column chunks keeps too few loads in flight when
// the rows are short).  `w` holds the wave's first item (item `wave`),
// loaded by the caller before its wait; later items come from the
// workgroup's LDS counter.  fn(row, sum_row, sum_row_plus_1) per row pair,
// called by lane 0.
template <int NR, int NC, typename Fn>
__device__ __forceinline__ void rows_matvec(SharedState &sh, u32x4 (&w)[NR][NC], const uint16_t *mat, size_t ld,
                                            int col0, const u32x4 *x, int r0, int nrows, Fn fn) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int nitems = (nrows + NR - 1) / NR;
    for (int it = wave; it < nitems; it = next_local_item(sh, lane)) {
        const int row = r0 + it * NR, nv = min(NR, nrows - it * NR);  // even, uniform
        if (it != wave) load_rows_upto<NR, NC>(w, mat, ld, row, nv, col0, lane);
        float acc[NR];
#pragma unroll
        for (int i = 0; i < NR; ++i) {
            acc[i] = 0.f;
            if (i < nv) {
#pragma unroll
                for (int k = 0; k < NC; ++k) acc[i] = dot8(w[i][k], x[k * 64 + lane], acc[i]);
                acc[i] = wave_sum(acc[i]);
            }
        }
        if (lane == 0) {
#pragma unroll
            for (int i = 0; i < NR; i += 2)
                if (i < nv) fn(row + i, acc[i], acc[i + 1]);
        }
    }
}

// NR for NC chunks per row: about 16-24 loads per lane per item.
template <int NC>
struct LmRows {
    static constexpr int kNR = NC <= 2 ? 8 : NC <= 6 ? 4 : 2;
};

// ---- opcode 7: Mixtral_RMS_LM_Head  (python_vm.py:321-345) ----------------

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));

// logits[r] += bf16(W[r, cols] . normed[cols]) for a pair of rows at a time:
// one packed bf16 atomic add per pair (rows are even-aligned).
__device__ __forceinline__ void lm_atomic_pair(uint16_t *logits, int r, float sa, float sb) {
    const bf16x2_t v = {__builtin_bit_cast(__bf16, (uint16_t)f2bf(sa)), __builtin_bit_cast(__bf16, (uint16_t)f2bf(sb))};
    __builtin_amdgcn_global_atomic_fadd_v2bf16((__attribute__((address_space(1))) bf16x2_t *)(logits + r), v);
}

// The instruction's rows in items of LmRows<NC> rows, the first item of
// each wave loaded before the wait (the weights do not depend on it).
template <int NC>
__device__ __forceinline__ bool lm_head_rows(kp_c &p, SharedState &sh, u32x4 *act, const Ctx &c,
                                             int32_t *tim, int r0, int nrows, int col0) {
    attn_c &a = attn_of(p);
    const int last = p.num_layers - 1;
    constexpr int NR = LmRows<NC>::kNR;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    u32x4 w[NR][NC];
    if (p.late_loads && !wait_ge(p, sh, bar_at(p, last, 6), p.down_arrivals, c, 7, last)) return false;
    stamp(tim, MK_TEVENT_FIRST_LOAD);
    if (wave * NR < nrows) load_rows_upto<NR, NC>(w, a.lm_head, (size_t)p.H, r0 + wave * NR, min(NR, nrows - wave * NR), col0, lane);
    stamp(tim, MK_TEVENT_AT_GMEM_WAIT);
    if (!p.late_loads && !wait_ge(p, sh, bar_at(p, last, 6), p.down_arrivals, c, 7, last)) return false;
    stamp(tim, MK_TEVENT_DONE_GMEM_WAIT);
    rms_to_lds(p, sh, act, a.lm_norm);
    rows_matvec<NR, NC>(sh, w, a.lm_head, (size_t)p.H, col0, act + (col0 >> 3), r0, nrows,
                        [&](int r, float sa, float sb) { lm_atomic_pair(a.logits, r, sa, sb); });
    drain_and_sync();
    stamp(tim, MK_TEVENT_DONE_GMEM_STORE);
    return true;
}

__device__ __forceinline__ bool op_lm_head(kp_c &p, SharedState &sh, u32x4 *act, ins_t *ins, const Ctx &c,
                           int32_t *tim) {
    const int b0 = __builtin_amdgcn_readfirstlane(ins[1]);
    const int b1 = __builtin_amdgcn_readfirstlane(ins[2]);
    const int red = __builtin_amdgcn_readfirstlane(ins[3]);
    const int last = p.num_layers - 1;
    if (!need_attention(p, c, 7, last)) return false;
    attn_c &a = attn_of(p);  // valid: attention tensors are present
    if (b0 < 0 || b1 < b0 || (int64_t)b1 * a.lm_bs > a.V || red < 0 || (int64_t)(red + 1) * a.lm_red > p.H) {
        report_error(p, MK_ERR_BAD_INSTRUCTION, c, 7, last, b0, b1);
        return false;
    }
    if (threadIdx.x == 0) sh.next_item = kWaves;
    const int col0 = red * a.lm_red;
    const int r0 = b0 * a.lm_bs, nrows = (b1 - b0) * a.lm_bs;
    switch (a.lm_red / kChunkElems) {
    case 1: return lm_head_rows<1>(p, sh, act, c, tim, r0, nrows, col0);
    case 2: return lm_head_rows<2>(p, sh, act, c, tim, r0, nrows, col0);
    case 3: return lm_head_rows<3>(p, sh, act, c, tim, r0, nrows, col0);
    case 4: return lm_head_rows<4>(p, sh, act, c, tim, r0, nrows, col0);
    default: break;
    }
    stamp(tim, MK_TEVENT_AT_GMEM_WAIT);
    if (!wait_ge(p, sh, bar_at(p, last, 6), p.down_arrivals, c, 7, last)) return false;
    stamp(tim, MK_TEVENT_DONE_GMEM_WAIT);
    rms_to_lds(p, sh, act, a.lm_norm);
    stamp(tim, MK_TEVENT_FIRST_LOAD);
    // longer reduction blocks: a row pair per item
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    for (int it = wave; 2 * it < nrows; it = next_local_item(sh, lane)) {
        const int ra = r0 + 2 * it;
        float aa = 0.f, ab = 0.f;
        dot_pair(a.lm_head + (size_t)ra * p.H + col0, a.lm_head + (size_t)(ra + 1) * p.H + col0, act + (col0 >> 3),
                 act + (col0 >> 3), a.lm_red / kChunkElems, lane, aa, ab);
        aa = wave_sum(aa);
        ab = wave_sum(ab);
        if (lane == 0) lm_atomic_pair(a.logits, ra, aa, ab);
    }
    drain_and_sync();
    stamp(tim, MK_TEVENT_DONE_GMEM_STORE);
    return true;
}

// ---------------------------------------------------------------------------
// the persistent interpreter
// ---------------------------------------------------------------------------

// kAttn: whether opcodes 1-4 and 7 are compiled in.  The MoE-only variant
// keeps the register allocation of the opcode 5/6 streaming loops free of
// the attention code's live ranges; launches without attention tensors use
// it.
// ---------------------------------------------------------------------------
// dense (Llama) opcodes 5-7  (lat/python_vm.py:83-196)
// ---------------------------------------------------------------------------

// Opcode 5, LayerNormDoubleMatVecSiLU [5, layer, n, block...]: RMSNorm with
// the MLP norm, then for each listed block of up_gate_proj_block_size rows
// silu_out[r] = bf16(bf16(silu(bf16 g)) * bf16 u), g and u the gate and up
// rows dotted with the normed vector; one arrival per block on [l][4][0].
// The dense weights are the one-expert case of the opcode-5 item.
__device__ __forceinline__ bool op_dense_upgate(kp_c &p, SharedState &sh, u32x4 *act, ins_t *ins,
                                                const Ctx &c, int32_t *tim) {
    const int layer = __builtin_amdgcn_readfirstlane(ins[1]);
    const int n = __builtin_amdgcn_readfirstlane(ins[2]);
    const int nblocks = p.F / p.expert_bs;
    bool bad = layer < 0 || layer >= p.num_layers || n < 0 || n > MK_INTS_PER_INSTRUCTION - 3;
    for (int i = 0; !bad && i < n; ++i) {
        const int b = __builtin_amdgcn_readfirstlane(ins[3 + i]);
        bad = b < 0 || b >= nblocks;
    }
    if (bad) {
        report_error(p, MK_ERR_BAD_INSTRUCTION, c, 5, layer, n, nblocks);
        return false;
    }
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int items = n * p.expert_bs, nc = p.H / kChunkElems;
    // items [0, S) staged in LDS: by the preceding opcode 4 (which left
    // sh.stage_slot / sh.stage_n set before its barriers), else here
    const bool pre_staged = __builtin_amdgcn_readfirstlane(sh.stage_slot) == c.slot;
    const int S = pre_staged ? __builtin_amdgcn_readfirstlane(sh.stage_n)
                             : stage_dense_upgate(p, sh, act, ins, c.slot, layer, false);
    if (threadIdx.x == 0) sh.next_item = S + kWaves;
    // each wave's first item from HBM (its gate and up rows) is loaded
    // before the wait: the weights do not depend on it (issued after the
    // wait instead, to stream while the staged items are computed, it
    // measured 7 % slower per decode step)
    const int ia = S + wave;
    PairAhead pre;
    auto load_ahead = [&]() {
        if (ia < items) {
            const int k = ia / p.expert_bs;
            const int row = __builtin_amdgcn_readfirstlane(ins[3 + k]) * p.expert_bs + ia - k * p.expert_bs;
            const size_t off = ((size_t)layer * p.F + row) * (size_t)p.H;
            const u32x4 *wg = reinterpret_cast<const u32x4 *>(p.gate + off) + lane;
            const u32x4 *wu = reinterpret_cast<const u32x4 *>(p.up + off) + lane;
#pragma unroll
            for (int i = 0; i < kAheadChunks; ++i)
                if (i < nc) {
                    pre.a[i] = load_stream(wg + i * 64);
                    pre.b[i] = load_stream(wu + i * 64);
                }
        }
    };
    auto wait = [&] { return wait_ge(p, sh, bar_at(p, layer, 4), p.H / p.oproj_bs, c, 5, layer); };
    if (p.late_loads && !wait()) return false;
    stamp(tim, MK_TEVENT_FIRST_LOAD);
    load_ahead();
    stamp(tim, MK_TEVENT_AT_GMEM_WAIT);
    if (!p.late_loads && !wait()) return false;
    stamp(tim, MK_TEVENT_DONE_GMEM_WAIT);
    if (threadIdx.x == 0) {
        sh.stage_slot = -1;  // every thread has read it (the wait ends in barriers)
        sh.route_layer = layer;  // this layer's O projection is complete: its residual rows are final
    }
    rms_to_lds(p, sh, act, p.ffn_ln + (size_t)layer * p.H);
    for (int it = wave; it < S; it += kWaves) {  // the staged items
        const int k = it / p.expert_bs;
        const int row = __builtin_amdgcn_readfirstlane(ins[3 + k]) * p.expert_bs + it - k * p.expert_bs;
        const u32x4 *sg = act + p.stage_off16 + (2 * it) * nc * 64 + lane;
        const u32x4 *su = sg + nc * 64;
        float ag = 0.f, au = 0.f;
        for (int ch = 0; ch < nc; ++ch) {
            ag = dot8(sg[ch * 64], act[ch * 64 + lane], ag);
            au = dot8(su[ch * 64], act[ch * 64 + lane], au);
        }
        silu_store(p, 0, row, wave_sum(ag), wave_sum(au), lane);
    }
    if (ia < items) {  // the item loaded ahead
        const int k = ia / p.expert_bs;
        const int row = __builtin_amdgcn_readfirstlane(ins[3 + k]) * p.expert_bs + ia - k * p.expert_bs;
        float ag = 0.f, au = 0.f;
#pragma unroll
        for (int i = 0; i < kAheadChunks; ++i)
            if (i < nc) {
                ag = dot8(pre.a[i], act[i * 64 + lane], ag);
                au = dot8(pre.b[i], act[i * 64 + lane], au);
            }
        if (nc > kAheadChunks) {
            const size_t off = ((size_t)layer * p.F + row) * (size_t)p.H + kAheadChunks * kChunkElems;
            dot_pair(p.gate + off, p.up + off, act + kAheadChunks * 64, act + kAheadChunks * 64, nc - kAheadChunks,
                     lane, ag, au);
        }
        silu_store(p, 0, row, wave_sum(ag), wave_sum(au), lane);
    }
    for (int it = next_local_item(sh, lane); it < items; it = next_local_item(sh, lane)) {
        const int k = it / p.expert_bs;
        const int row = __builtin_amdgcn_readfirstlane(ins[3 + k]) * p.expert_bs + it - k * p.expert_bs;
        upgate_item(p, act, layer, row, 1, 0, 0, 0, lane);
    }
    drain_and_sync();
    arrive(p, bar_at(p, layer, 5), n);
    stamp(tim, MK_TEVENT_DONE_GMEM_STORE);
    return true;
}

// NR rows x NC chunks of a row-major bf16 matrix (row stride ld, columns
// from col0), 16 bytes per lane per (row, chunk): all NR * NC loads are
// issued before any is used.
template <int NR, int NC>
__device__ __forceinline__ void load_rows(u32x4 (&w)[NR][NC], const uint16_t *mat, size_t ld, int row, int col0,
                                          int lane) {
#pragma unroll
    for (int i = 0; i < NR; ++i)
#pragma unroll
        for (int c = 0; c < NC; ++c)
            w[i][c] = load_stream(reinterpret_cast<const u32x4 *>(mat + (size_t)(row + i) * ld + col0) + c * 64 + lane);
}

// Opcode 6, DownProjResidual [6, layer, start, end, red]: rows
// [start, end) * down_proj_block_size of the down projection, columns
// [red, red + 1) * red_cols, dotted with those columns of silu_out; each row
// pair is added into hidden with one packed bf16 atomic (the column chunks
// of a row run on different workgroups), h = bf16(h + bf16(partial)).
// Arrival end - start on [l][5][0].  Items are NR rows x NC = red_cols / 512
// chunks (16 loads per lane); each wave's first item is loaded before the
// wait on opcode 5, since the weights do not depend on it.
template <int NR, int NC>
__device__ __forceinline__ bool dense_down_rows(kp_c &p, SharedState &sh, u32x4 *act, const Ctx &c,
                                                int32_t *tim, int layer, int b0, int b1, int red) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int R = p.red_cols, col0 = red * R;
    const int r0 = b0 * p.down_bs, nitems = (b1 - b0) * p.down_bs / NR;
    const uint16_t *wm = p.down + (size_t)layer * p.H * p.F;
    u32x4 w[NR][NC];
    auto wait = [&] { return wait_ge(p, sh, bar_at(p, layer, 5), p.F / p.expert_bs, c, 6, layer); };
    if (p.late_loads && !wait()) return false;
    stamp(tim, MK_TEVENT_FIRST_LOAD);
    if (wave < nitems) load_rows<NR, NC>(w, wm, (size_t)p.F, r0 + wave * NR, col0, lane);
    stamp(tim, MK_TEVENT_AT_GMEM_WAIT);
    if (!p.late_loads && !wait()) return false;
    stamp(tim, MK_TEVENT_DONE_GMEM_WAIT);
    for (int v = threadIdx.x; v < (R >> 3); v += kThreads) act[v] = ld_dev128(p.silu, (uint32_t)(col0 + v * 8) * 2u);
    __syncthreads();
    for (int it = wave; it < nitems; it = next_local_item(sh, lane)) {
        const int row = r0 + it * NR;
        if (it != wave) load_rows<NR, NC>(w, wm, (size_t)p.F, row, col0, lane);
        float acc[NR];
#pragma unroll
        for (int i = 0; i < NR; ++i) {
            acc[i] = 0.f;
#pragma unroll
            for (int k = 0; k < NC; ++k) acc[i] = dot8(w[i][k], act[k * 64 + lane], acc[i]);
            acc[i] = wave_sum(acc[i]);
        }
        if (lane == 0) {
#pragma unroll
            for (int i = 0; i < NR; i += 2) {
                const bf16x2_t v = {__builtin_bit_cast(__bf16, (uint16_t)f2bf(acc[i])),
                                    __builtin_bit_cast(__bf16, (uint16_t)f2bf(acc[i + 1]))};
                __builtin_amdgcn_global_atomic_fadd_v2bf16(
                    (__attribute__((address_space(1))) bf16x2_t *)(p.hidden + row + i), v);
            }
        }
    }
    drain_and_sync();
    arrive(p, bar_at(p, layer, 6), b1 - b0);
    stamp(tim, MK_TEVENT_DONE_GMEM_STORE);
    return true;
}

// Opcode 6 when the column chunk is all of F (matvec_reduction_size == F):
// every row has one writer, so h = bf16(h + bf16(W[r] . silu)) is a plain
// coherent read-modify-write in python_vm's order, with no atomics, and a
// relaunch is bit-identical.  An item is one full row of
// [start, end) * down_proj_block_size (nc chunks, up to kSegChunks loads per
// lane in flight), stored by its wave as soon as its sum is known, so only
// the last item's store is outstanding at the end.  The first item of each
// wave (its first kSegChunks chunks) is loaded before the wait, the rows
// after those (as many as the launch's LDS holds after the SiLU row) are
// streamed into LDS by waves 1.. (wave 0 polls), and, when this
// workgroup's opcode 5 already passed the O-proj wait (the residual rows
// are final then), so are the first kRowBatch residual rows.  After the
// wait only the SiLU row is read from memory before the sums.
__device__ __forceinline__ bool dense_down_full(kp_c &p, SharedState &sh, u32x4 *act, const Ctx &c,
                                                int32_t *tim, int layer, int b0, int b1) {
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int r0 = b0 * p.down_bs, nrows = (b1 - b0) * p.down_bs;
    const int nc = p.F / kChunkElems;
    const uint16_t *wm = p.down + (size_t)layer * p.H * p.F;
    const int nearly = min(nrows, kRowBatch);  // rows whose residual is read before the wait
    auto wait = [&] { return wait_ge(p, sh, bar_at(p, layer, 5), p.F / p.expert_bs, c, 6, layer); };
    if (p.late_loads && !wait()) return false;
    RowRegs<kSegChunks> pre;  // up to a whole first row per wave (16 KiB), as many loads as a later item
    stamp(tim, MK_TEVENT_FIRST_LOAD);
    if (wave < nrows)
        load_row<kSegChunks>(pre, reinterpret_cast<const u32x4 *>(wm + (size_t)(r0 + wave) * p.F) + lane,
                             min(nc, kSegChunks));
    const bool hfinal = !p.late_loads && __builtin_amdgcn_readfirstlane(sh.route_layer) == layer;
    uint32_t hpre = 0;
    if (hfinal && tid < nearly) hpre = ld_dev16(p.hidden + r0 + tid);
    // rows kWaves .. kWaves + nst - 1, row-major 512-column chunks in lane
    // order after the SiLU row
    const int soff16 = ((p.F * 2 + 1023) / 1024) * 64;  // u32x4 units
    const int nst = p.late_loads ? 0 : min(max(nrows - kWaves, 0), max(p.lds_bytes / 16 - soff16, 0) / (nc * 64));
    if (wave >= 1)
        for (int q = wave - 1; q < nst; q += kWaves - 1) {
            const u32x4 *w = reinterpret_cast<const u32x4 *>(wm + (size_t)(r0 + kWaves + q) * p.F) + lane;
            for (int ch = 0; ch < nc; ++ch)
                __builtin_amdgcn_global_load_lds((global_void_t *)(w + ch * 64),
                                                 (lds_void_t *)(act + soff16 + (q * nc + ch) * 64), 16, 0, 0);
        }
    stamp(tim, MK_TEVENT_AT_GMEM_WAIT);
    if (!p.late_loads && !wait()) return false;
    stamp(tim, MK_TEVENT_DONE_GMEM_WAIT);
    uint32_t *hrow = reinterpret_cast<uint32_t *>(sh.part);  // the residual rows read early
    if (hfinal && tid < nearly) hrow[tid] = hpre;
    for (int v = tid; v < (p.F >> 3); v += kThreads) act[v] = ld_dev128(p.silu, (uint32_t)v * 16u);
    __builtin_amdgcn_s_waitcnt(kVmcntZero);  // this wave's staged rows have landed too
    __syncthreads();
    // the rest of row r0 + it from chunk `done` on, added to acc
    auto row_rest = [&](int it, int done, float acc) {
        const u32x4 *w = reinterpret_cast<const u32x4 *>(wm + (size_t)(r0 + it) * p.F) + lane;
        while (done < nc) {
            const int n = min(nc - done, kSegChunks);
            RowRegs<kSegChunks> r;
            load_row<kSegChunks>(r, w + done * 64, n);
            acc = dot_row_regs<kSegChunks>(r, act + lane + done * 64, n, acc);
            done += n;
        }
        return acc;
    };
    auto store_row = [&](int it, float acc) {  // lane 0
        uint16_t *hp = p.hidden + r0 + it;
        const uint32_t h = hfinal && it < nearly ? hrow[it] : ld_dev16(hp);
        st_dev16(hp, f2bf(bf2f(h) + rbf(acc)));
    };
    // the items loaded before the wait (outside the item loop, so their
    // registers are free again for the later items)
    if (wave < nrows) {
        const int n = min(nc, kSegChunks);
        const float acc = wave_sum(row_rest(wave, n, dot_row_regs<kSegChunks>(pre, act + lane, n, 0.f)));
        if (lane == 0) store_row(wave, acc);
    }
    for (int it = next_local_item(sh, lane); it < nrows; it = next_local_item(sh, lane)) {
        float acc = 0.f;
        if (it - kWaves < nst) {  // the same chunk order as row_rest
            const u32x4 *s = act + soff16 + (it - kWaves) * nc * 64 + lane;
            for (int ch = 0; ch < nc; ++ch) acc = dot8(s[ch * 64], act[lane + ch * 64], acc);
        } else {
            acc = row_rest(it, 0, 0.f);
        }
        acc = wave_sum(acc);
        if (lane == 0) store_row(it, acc);
    }
    drain_and_sync();
    arrive(p, bar_at(p, layer, 6), b1 - b0);
    stamp(tim, MK_TEVENT_DONE_GMEM_STORE);
    return true;
}

__device__ __forceinline__ bool op_dense_down(kp_c &p, SharedState &sh, u32x4 *act, ins_t *ins,
                                              const Ctx &c, int32_t *tim) {
    const int layer = __builtin_amdgcn_readfirstlane(ins[1]);
    const int b0 = __builtin_amdgcn_readfirstlane(ins[2]);
    const int b1 = __builtin_amdgcn_readfirstlane(ins[3]);
    const int red = __builtin_amdgcn_readfirstlane(ins[4]);
    if (layer < 0 || layer >= p.num_layers || b0 < 0 || b1 < b0 || (int64_t)b1 * p.down_bs > p.H || red < 0 ||
        (int64_t)(red + 1) * p.red_cols > p.F) {
        report_error(p, MK_ERR_BAD_INSTRUCTION, c, 6, layer, b0, red);
        return false;
    }
    if (threadIdx.x == 0) sh.next_item = kWaves;
    if (p.red_cols == p.F) return dense_down_full(p, sh, act, c, tim, layer, b0, b1);
    // the host admits red_cols of 1, 2, 4 or 8 chunks and even block sizes
    // that the row group divides
    switch (p.red_cols / kChunkElems) {
    case 1: return dense_down_rows<16, 1>(p, sh, act, c, tim, layer, b0, b1, red);
    case 2: return dense_down_rows<8, 2>(p, sh, act, c, tim, layer, b0, b1, red);
    case 4: return dense_down_rows<4, 4>(p, sh, act, c, tim, layer, b0, b1, red);
    default: return dense_down_rows<2, 8>(p, sh, act, c, tim, layer, b0, b1, red);
    }
}

// Running argmax in torch.argmax's order: NaN above every number, then the
// larger value, then the lower index (idx < 0: empty).
struct ArgBest {
    float v;
    int idx;
    bool nan;
};

__device__ __forceinline__ bool arg_better(const ArgBest &b, const ArgBest &a) {
    if (b.idx < 0) return false;
    if (a.idx < 0) return true;
    if (a.nan || b.nan) return a.nan && b.nan ? b.idx < a.idx : b.nan;
    return b.v > a.v || (b.v == a.v && b.idx < a.idx);
}

__device__ __forceinline__ void arg_take(ArgBest &a, float v, int idx) {
    const ArgBest b{v, idx, v != v};
    if (arg_better(b, a)) a = b;
}

// The waves' best logits of a dense LM-head instruction (one ArgBest per
// wave, in lane 0) merged into the workgroup's running best (sh.lm_v,
// sh.lm_idx), which kernel_exit publishes for the exit argmax.  Ends with a
// workgroup barrier.
__device__ __forceinline__ void lm_best_merge(SharedState &sh, const ArgBest &wb) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    if (lane == 0) {
        sh.red[wave] = wb.v;
        sh.wave_cnt[wave] = wb.idx;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        ArgBest r{sh.lm_v, sh.lm_idx, sh.lm_v != sh.lm_v};
        for (int w = 0; w < kWaves; ++w) {
            const ArgBest o{sh.red[w], sh.wave_cnt[w], sh.red[w] != sh.red[w]};
            if (arg_better(o, r)) r = o;
        }
        sh.lm_v = r.v;
        sh.lm_idx = r.idx;
    }
    __syncthreads();
}

// Opcode 7, RMS_LM_Head [7, start, end]: RMSNorm with the LM-head norm, then
// logits[r] = bf16(W[r] . normed) over all hidden columns for rows
// [start, end) * lm_head_block_size, stored (not accumulated) with one
// 32-bit coherent store per row pair.
template <int NC>
__device__ __forceinline__ bool dense_lm_head_rows(kp_c &p, SharedState &sh, u32x4 *act, const Ctx &c,
                                                   int32_t *tim, int r0, int nrows) {
    attn_c &a = attn_of(p);
    const int last = p.num_layers - 1;
    constexpr int NR = LmRows<NC>::kNR;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    u32x4 w[NR][NC];
    if (p.late_loads && !wait_ge(p, sh, bar_at(p, last, 6), p.down_arrivals, c, 7, last)) return false;
    stamp(tim, MK_TEVENT_FIRST_LOAD);
    if (wave * NR < nrows) load_rows_upto<NR, NC>(w, a.lm_head, (size_t)p.H, r0 + wave * NR, min(NR, nrows - wave * NR), 0, lane);
    stamp(tim, MK_TEVENT_AT_GMEM_WAIT);
    if (!p.late_loads && !wait_ge(p, sh, bar_at(p, last, 6), p.down_arrivals, c, 7, last)) return false;
    stamp(tim, MK_TEVENT_DONE_GMEM_WAIT);
    rms_to_lds(p, sh, act, a.lm_norm);
    ArgBest wb{0.f, -1, false};  // lane 0: the wave's best stored logit
    rows_matvec<NR, NC>(sh, w, a.lm_head, (size_t)p.H, 0, act, r0, nrows, [&](int r, float sa, float sb) {
        const uint32_t ba = f2bf(sa), bb = f2bf(sb);
        st_dev32(a.logits + r, ba | (bb << 16));
        arg_take(wb, bf2f(ba), r);
        arg_take(wb, bf2f(bb), r + 1);
    });
    drain_and_sync();
    if (p.lm_cand != nullptr) lm_best_merge(sh, wb);
    stamp(tim, MK_TEVENT_DONE_GMEM_STORE);
    return true;
}

__device__ __forceinline__ bool op_dense_lm_head(kp_c &p, SharedState &sh, u32x4 *act, ins_t *ins,
                                                 const Ctx &c, int32_t *tim) {
    const int b0 = __builtin_amdgcn_readfirstlane(ins[1]);
    const int b1 = __builtin_amdgcn_readfirstlane(ins[2]);
    const int last = p.num_layers - 1;
    if (!need_attention(p, c, 7, last)) return false;
    attn_c &a = attn_of(p);  // valid: attention tensors are present
    if (b0 < 0 || b1 < b0 || (int64_t)b1 * a.lm_bs > a.V) {
        report_error(p, MK_ERR_BAD_INSTRUCTION, c, 7, last, b0, b1);
        return false;
    }
    if (threadIdx.x == 0) sh.next_item = kWaves;
    const int r0 = b0 * a.lm_bs, nrows = (b1 - b0) * a.lm_bs;
    switch (p.H / kChunkElems) {
    case 2: return dense_lm_head_rows<2>(p, sh, act, c, tim, r0, nrows);
    case 3: return dense_lm_head_rows<3>(p, sh, act, c, tim, r0, nrows);
    case 4: return dense_lm_head_rows<4>(p, sh, act, c, tim, r0, nrows);
    case 5: return dense_lm_head_rows<5>(p, sh, act, c, tim, r0, nrows);
    case 6: return dense_lm_head_rows<6>(p, sh, act, c, tim, r0, nrows);
    case 8: return dense_lm_head_rows<8>(p, sh, act, c, tim, r0, nrows);
    default: break;
    }
    stamp(tim, MK_TEVENT_AT_GMEM_WAIT);
    if (!wait_ge(p, sh, bar_at(p, last, 6), p.down_arrivals, c, 7, last)) return false;
    stamp(tim, MK_TEVENT_DONE_GMEM_WAIT);
    rms_to_lds(p, sh, act, a.lm_norm);
    stamp(tim, MK_TEVENT_FIRST_LOAD);
    // other hidden sizes: a row pair per item
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    ArgBest wb{0.f, -1, false};  // lane 0: the wave's best stored logit
    for (int it = wave; 2 * it < nrows; it = next_local_item(sh, lane)) {
        const int ra = r0 + 2 * it;
        float aa = 0.f, ab = 0.f;
        dot_pair(a.lm_head + (size_t)ra * p.H, a.lm_head + (size_t)(ra + 1) * p.H, act, act, p.H / kChunkElems, lane,
                 aa, ab);
        aa = wave_sum(aa);
        ab = wave_sum(ab);
        if (lane == 0) {
            const uint32_t ba = f2bf(aa), bb = f2bf(ab);
            st_dev32(a.logits + ra, ba | (bb << 16));
            arg_take(wb, bf2f(ba), ra);
            arg_take(wb, bf2f(bb), ra + 1);
        }
    }
    drain_and_sync();
    if (p.lm_cand != nullptr) lm_best_merge(sh, wb);
    stamp(tim, MK_TEVENT_DONE_GMEM_STORE);
    return true;
}

// Decode-driver tail of a launch, run by the last workgroup to exit (every
// LM-head instruction has completed by then): argmax over the V logits,
// written to p.argmax_out, and with p.next_embed the embedding row of that
// token copied into hidden.  Replaces the generator's torch.argmax and
// embedding lookup between launches (megakernels/generators.py:121-145).
__device__ __forceinline__ void exit_argmax(kp_c &p, SharedState &sh) {
    attn_c &a = attn_of(p);
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int V = a.V, nv = V >> 3;
    ArgBest best{0.f, -1, false};
    if (p.lm_cand != nullptr) {
        // every workgroup's best stored logit (kernel_exit published them
        // before counting out)
        for (int w = tid; w < (int)gridDim.x; w += kThreads) {
            const float v = __uint_as_float(ld_dev32(p.lm_cand + 2 * w));
            const ArgBest o{v, (int)ld_dev32(p.lm_cand + 2 * w + 1), v != v};
            if (arg_better(o, best)) best = o;
        }
    } else {
        // 16 B per lane, up to 16 loads in flight per thread (one round trip
        // for up to 64 K logits); a thread visits its indices in increasing
        // order, so a later value replaces its best only if it is larger, or
        // the first NaN
        constexpr int kArgLoads = 16;
        for (int base = 0; base < nv; base += kArgLoads * kThreads) {
            u32x4 x[kArgLoads];
#pragma unroll
            for (int k = 0; k < kArgLoads; ++k) {
                const int v = base + k * kThreads + tid;
                if (v < nv) x[k] = ld_dev128(a.logits, (uint32_t)v * 16u);
            }
#pragma unroll
            for (int k = 0; k < kArgLoads; ++k) {
                const int v = base + k * kThreads + tid;
                if (v < nv) {
                    const uint32_t w[4] = {x[k].x, x[k].y, x[k].z, x[k].w};
#pragma unroll
                    for (int j = 0; j < 8; ++j) {
                        const float f = bf2f((w[j >> 1] >> (16 * (j & 1))) & 0xffffu);
                        const int i = 8 * v + j;
                        const bool take = !best.nan && (f != f || best.idx < 0 || f > best.v);
                        best.nan = best.nan || f != f;
                        best.v = take ? f : best.v;
                        best.idx = take ? i : best.idx;
                    }
                }
            }
        }
        for (int i = 8 * nv + tid; i < V; i += kThreads) arg_take(best, bf2f(ld_dev16(a.logits + i)), i);
    }
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) {
        const ArgBest o{__shfl_xor(best.v, m), __shfl_xor(best.idx, m), __shfl_xor((int)best.nan, m) != 0};
        if (arg_better(o, best)) best = o;
    }
    if (lane == 0) {
        sh.red[wave] = best.v;
        sh.wave_cnt[wave] = best.idx;
        sh.red_ss[wave] = best.nan ? 1.f : 0.f;
    }
    __syncthreads();
    if (tid == 0) {
        ArgBest r{0.f, -1, false};
        for (int w = 0; w < kWaves; ++w) {
            const ArgBest o{sh.red[w], sh.wave_cnt[w], sh.red_ss[w] != 0.f};
            if (arg_better(o, r)) r = o;
        }
        *p.argmax_out = (int64_t)r.idx;
        sh.flag = r.idx;
    }
    __syncthreads();
    if (p.next_embed != nullptr) {
        const int tok = sh.flag;
        const u32x4 *src = reinterpret_cast<const u32x4 *>(p.next_embed + (size_t)tok * p.H);
        u32x4 *dst = reinterpret_cast<u32x4 *>(p.hidden);
        for (int v = tid; v < (p.H >> 3); v += kThreads) dst[v] = src[v];
    }
}

// Zero n 32-bit words at p (4-byte aligned) with the workgroup: 16-byte
// stores from the first 16-byte boundary on.
__device__ __forceinline__ void zero_words(uint32_t *p, size_t n) {
    const size_t head = min(n, (size_t)((16u - (reinterpret_cast<uintptr_t>(p) & 15u)) & 15u) / 4);
    if (threadIdx.x < head) p[threadIdx.x] = 0u;
    u32x4 *v = reinterpret_cast<u32x4 *>(p + head);
    const size_t nv = (n - head) / 4;
    for (size_t i = threadIdx.x; i < nv; i += kThreads) v[i] = u32x4{0u, 0u, 0u, 0u};
    for (size_t i = head + nv * 4 + threadIdx.x; i < n; i += kThreads) p[i] = 0u;
}

// Exit protocol: the last workgroup out (failed or not) zeroes the
// work-sharing counters for the next launch, after the decode-driver tail
// when one was asked for.  Every other workgroup has finished all of its
// scratch accesses before it increments the counter.
__device__ __forceinline__ void kernel_exit(kp_c &p, SharedState &sh) {
    if (p.lm_cand != nullptr && threadIdx.x == 0) {
        st_dev32(p.lm_cand + 2 * blockIdx.x, __float_as_uint(sh.lm_v));
        st_dev32(p.lm_cand + 2 * blockIdx.x + 1, (uint32_t)sh.lm_idx);
    }
    drain_and_sync();
    if (threadIdx.x == 0) {
        const int prev = __hip_atomic_fetch_add(p.scratch, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        sh.flag = prev == (int)gridDim.x - 1;
    }
    __syncthreads();
    if (sh.flag) {
        if (p.argmax_out != nullptr && p.attn && !aborted(p)) exit_argmax(p, sh);
        // spread counters: their parts back into the barrier tensor (which
        // then holds what the reference's counters would), parts zeroed; a
        // launch that zeroes the barrier tensor for the next one only
        // zeroes the parts (stores, no round trip)
        if (p.spread != nullptr && p.reset_next > 0) {
            for (int row = threadIdx.x; row < p.spread_rows; row += kThreads)
#pragma unroll
                for (int k = 0; k < kSpread; ++k) st_dev32(p.spread + (size_t)k * p.spread_stride + row, 0u);
        } else if (p.spread != nullptr) {
            for (int row = threadIdx.x; row < p.spread_rows; row += kThreads) {
                int sum = 0;
#pragma unroll
                for (int k = 0; k < kSpread; ++k) {
                    int32_t *q = p.spread + (size_t)k * p.spread_stride + row;
                    sum += (int)ld_dev32(q);
                    st_dev32(q, 0u);
                }
                if (sum != 0) {
                    int32_t *b = p.bar + (size_t)row * p.bar_width;
                    st_dev32(b, ld_dev32(b) + (uint32_t)sum);
                }
            }
        }
        if (p.reset_next > 0) {
            // every other workgroup is done with the barriers, and the
            // argmax above has read the logits
            zero_words(reinterpret_cast<uint32_t *>(p.bar), (size_t)p.num_layers * p.bar_ops * p.bar_width);
            if (p.reset_next > 1 && p.attn) {
                attn_c &a = attn_of(p);
                zero_words(reinterpret_cast<uint32_t *>(a.logits), (size_t)(a.V >> 1));
                if ((a.V & 1) && threadIdx.x == 0) a.logits[a.V - 1] = 0;
            }
        }
        // work-sharing cursors, then the column-chunk counters
        zero_words(reinterpret_cast<uint32_t *>(p.scratch + kScratchSlotBase), (size_t)p.scratch_clear);
        drain_and_sync();
        if (threadIdx.x == 0) __hip_atomic_store(p.scratch, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
}

template <int kE, bool kAttn>
__global__ void __launch_bounds__(kThreads) mk_mixtral_kernel(KParams) {
    const uint64_t code = kernel_code_base();
    kp_c &p = kparams();
    extern __shared__ u32x4 act[];
    __shared__ SharedState sh;
    if (threadIdx.x == 0) {
        sh.route_layer = -1;
        sh.stage_slot = -1;
        sh.ostage_slot = -1;
        sh.lm_v = 0.f;
        sh.lm_idx = -1;
    }
    __syncthreads();

    const int w = blockIdx.x;
    for (int q = 0; q < p.queue_len; ++q) {
        const size_t slot = (size_t)w * p.queue_len + q;
        ins_t *ins = (ins_t *)(p.instructions) + slot * MK_INTS_PER_INSTRUCTION;
        int32_t *tim = p.timings != nullptr ? p.timings + slot * MK_TIMING_SLOTS : nullptr;
        const int op = __builtin_amdgcn_readfirstlane(ins[0]);
        const Ctx c{w, q};
        stamp(tim, MK_TEVENT_START);
        touch_next_instruction(p, sh, ins, q);
        code_prefetch(p, sh, code, q);
        bool ok = true;
        switch (op) {
        case 0: break;
        case 5: {
            int consumed = 1;
            handler_prefetch(p, sh, code);
            ok = op_rms_router_upgate<kE, kAttn>(p, sh, act, ins, c, tim, consumed);
            q += consumed - 1;
            break;
        }
        case 6:
            handler_prefetch(p, sh, code);
            ok = op_expert_downproj<kE == 8 && !kAttn>(p, sh, act, ins, c, tim);
            break;
        case 8:
            handler_prefetch(p, sh, code);
            ok = op_predict<kE>(p, sh, act, ins, c, tim);
            break;
        case 1:
        case 2:
        case 3:
        case 4:
        case 7:
            if constexpr (kAttn) {
                // the prefetch in each branch: its program counter is where
                // that handler's code starts
                if (op == 1) {
                    handler_prefetch(p, sh, code);
                    ok = op_qkv(p, sh, act, ins, c, tim);
                } else if (op == 2) {
                    handler_prefetch(p, sh, code);
                    ok = op_partial_attn(p, sh, act, ins, c, tim);
                } else if (op == 3) {
                    handler_prefetch(p, sh, code);
                    ok = op_attn_reduction(p, sh, act, ins, c, tim);
                } else if (op == 4) {
                    handler_prefetch(p, sh, code);
                    ok = op_oproj(p, sh, act, ins, c, tim);
                } else {
                    handler_prefetch(p, sh, code);
                    ok = op_lm_head(p, sh, act, ins, c, tim);
                }
            } else {
                ok = need_attention(p, c, op, __builtin_amdgcn_readfirstlane(ins[1]));
            }
            break;
        default:
            report_error(p, MK_ERR_BAD_OPCODE, c, op, 0, 0, op);
            ok = false;
            break;
        }
        stamp(tim, MK_TEVENT_END);
        if (!ok) break;
    }

    kernel_exit(p, sh);
}

// Persistent kernel of the dense Llama VM (lat/ opcodes 1-7): the attention
// side is shared with the Mixtral kernel; opcodes 5-7 are the dense MLP and
// the LM head.
__global__ void __launch_bounds__(kThreads) mk_llama_kernel(KParams) {
    const uint64_t code = kernel_code_base();
    kp_c &p = kparams();
    extern __shared__ u32x4 act[];
    __shared__ SharedState sh;
    if (threadIdx.x == 0) {
        sh.route_layer = -1;
        sh.stage_slot = -1;
        sh.ostage_slot = -1;
        sh.lm_v = 0.f;
        sh.lm_idx = -1;
    }
    __syncthreads();

    const int w = blockIdx.x;
    for (int q = 0; q < p.queue_len; ++q) {
        const size_t slot = (size_t)w * p.queue_len + q;
        ins_t *ins = (ins_t *)(p.instructions) + slot * MK_INTS_PER_INSTRUCTION;
        int32_t *tim = p.timings != nullptr ? p.timings + slot * MK_TIMING_SLOTS : nullptr;
        const int op = __builtin_amdgcn_readfirstlane(ins[0]);
        const Ctx c{w, q};
        stamp(tim, MK_TEVENT_START);
        touch_next_instruction(p, sh, ins, q);
        code_prefetch(p, sh, code, q);
        bool ok = true;
        switch (op) {
        case 0: break;
        case 1: handler_prefetch(p, sh, code); ok = op_qkv(p, sh, act, ins, c, tim); break;
        case 2: handler_prefetch(p, sh, code); ok = op_partial_attn(p, sh, act, ins, c, tim); break;
        case 3: handler_prefetch(p, sh, code); ok = op_attn_reduction(p, sh, act, ins, c, tim); break;
        case 4: handler_prefetch(p, sh, code); ok = op_oproj(p, sh, act, ins, c, tim); break;
        case 5: handler_prefetch(p, sh, code); ok = op_dense_upgate(p, sh, act, ins, c, tim); break;
        case 6: handler_prefetch(p, sh, code); ok = op_dense_down(p, sh, act, ins, c, tim); break;
        case 7: handler_prefetch(p, sh, code); ok = op_dense_lm_head(p, sh, act, ins, c, tim); break;
        default:
            report_error(p, MK_ERR_BAD_OPCODE, c, op, 0, 0, op);
            ok = false;
            break;
        }
        stamp(tim, MK_TEVENT_END);
        if (!ok) break;
    }
    kernel_exit(p, sh);
}

// ---------------------------------------------------------------------------
// host side
// ---------------------------------------------------------------------------

constexpr int kMaxDevices = 64;

// Fixed scratch of mk_mixtral_launch_noalloc (2 MiB per device, held until
// the process ends): ints [0, kNoAllocStatusInts) are its status words when
// the caller passes none, the launch's scratch (exit counter, work-sharing
// cursors, column-chunk counters, spread counters) starts at
// kNoAllocBaseInts.  Every workgroup leaves through kernel_exit, whose last
// workgroup zeroes what the launch used, so each launch finds it zero (as
// the module loaded it).  Host code never passes `scratch` itself to a
// kernel: its address on a device comes from hipGetSymbolAddress
// (DeviceState::noalloc_scratch).
constexpr size_t kNoAllocScratchInts = (size_t)1 << 19;
constexpr size_t kNoAllocStatusInts = MK_STATUS_WORDS;
constexpr size_t kNoAllocBaseInts = 64;  // 256-byte aligned
static_assert(kNoAllocStatusInts <= kNoAllocBaseInts, "status words overlap the launch scratch");
static __device__ __align__(256) int32_t scratch[kNoAllocScratchInts];

// Library state per device.  The scratch buffer (exit counter, work-sharing
// cursors, column-chunk counters) and the status words are shared by every
// launch on the device, and a persistent kernel needs all of its workgroups
// resident at once, which two of them running together on one device cannot
// be promised.  So launches on one device run one after another: a launch on
// a stream other than the previous launch's first makes its stream wait for
// everything the previous one has queued (launch_mutex keeps the check, the
// scratch buffer and the launch together).
struct DeviceState {
    bool ready = false;
    int num_cus = 0;
    int max_lds = 0;
    int32_t *status = nullptr;
    int32_t *scratch = nullptr;
    size_t scratch_ints = 0;
    std::mutex launch_mutex;
    bool launched = false;
    hipStream_t last_stream = nullptr;
    hipEvent_t order_event = nullptr;
    // this device's copy of `scratch` (mk_mixtral_launch_noalloc), set once
    int32_t *noalloc_scratch = nullptr;
};

std::mutex g_mutex;
DeviceState g_devices[kMaxDevices];
thread_local int g_last_hip_error = 0;
thread_local const char *g_last_hip_site = "";

int hip_fail(hipError_t e, const char *site) {
    g_last_hip_error = (int)e;
    g_last_hip_site = site;
    return MK_ERR_HIP;
}

// `dev` must be the current device.  The device attributes are read once;
// the library-owned status words are allocated on the first call that asks
// for them (`with_status`), the no-allocation launch's fixed scratch is
// looked up on the first call that asks for it (`with_noalloc`).
int device_state(int dev, DeviceState **out, bool with_status = true, bool with_noalloc = false) {
    if (dev < 0 || dev >= kMaxDevices) return MK_ERR_INVALID_ARGUMENT;
    std::lock_guard<std::mutex> lock(g_mutex);
    DeviceState &st = g_devices[dev];
    hipError_t e;
    if (!st.ready) {
        e = hipDeviceGetAttribute(&st.num_cus, hipDeviceAttributeMultiprocessorCount, dev);
        if (e != hipSuccess) return hip_fail(e, "hipDeviceGetAttribute");
        e = hipDeviceGetAttribute(&st.max_lds, hipDeviceAttributeMaxSharedMemoryPerBlock, dev);
        if (e != hipSuccess) return hip_fail(e, "hipDeviceGetAttribute");
        st.ready = true;
    }
    if (with_status && st.status == nullptr) {
        int32_t *s = nullptr;
        e = hipMalloc(reinterpret_cast<void **>(&s), MK_STATUS_WORDS * sizeof(int32_t));
        if (e != hipSuccess) return hip_fail(e, "hipMalloc");
        e = hipMemset(s, 0, MK_STATUS_WORDS * sizeof(int32_t));
        if (e != hipSuccess) {
            (void)hipFree(s);
            return hip_fail(e, "hipMemset");
        }
        st.status = s;
    }
    if (with_noalloc && st.noalloc_scratch == nullptr) {
        // each device holds its own copy of the array, at its own address
        void *ptr = nullptr;
        e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
        if (e != hipSuccess || ptr == nullptr) return hip_fail(e != hipSuccess ? e : hipErrorInvalidSymbol,
                                                              "hipGetSymbolAddress");
        st.noalloc_scratch = static_cast<int32_t *>(ptr);
    }
    *out = &st;
    return MK_OK;
}

// Makes `device` current for the guard's lifetime.
struct DeviceGuard {
    int prev = -1;
    hipError_t err = hipSuccess;
    explicit DeviceGuard(int device) {
        err = hipGetDevice(&prev);
        if (err == hipSuccess && prev != device) err = hipSetDevice(device);
    }
    ~DeviceGuard() {
        int cur = -1;
        if (prev >= 0 && hipGetDevice(&cur) == hipSuccess && cur != prev) (void)hipSetDevice(prev);
    }
};

bool aligned16(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// The per-device scratch buffer holds at least `need` ints (exit counter and
// work-sharing cursors per instruction slot).
int ensure_scratch(DeviceState *st, size_t need) {
    if (need <= st->scratch_ints) return MK_OK;
    std::lock_guard<std::mutex> lock(g_mutex);
    if (need <= st->scratch_ints) return MK_OK;
    hipError_t e;
    size_t cap = st->scratch_ints ? st->scratch_ints : 4096;
    while (cap < need) cap *= 2;
    if (st->scratch != nullptr) {
        // kernels queued earlier may still use the old buffer
        if ((e = hipDeviceSynchronize()) != hipSuccess) return hip_fail(e, "hipDeviceSynchronize");
        if ((e = hipFree(st->scratch)) != hipSuccess) return hip_fail(e, "hipFree");
        st->scratch = nullptr;
        st->scratch_ints = 0;
    }
    if ((e = hipMalloc(reinterpret_cast<void **>(&st->scratch), cap * sizeof(int32_t))) != hipSuccess)
        return hip_fail(e, "hipMalloc");
    if ((e = hipMemset(st->scratch, 0, cap * sizeof(int32_t))) != hipSuccess) return hip_fail(e, "hipMemset");
    st->scratch_ints = cap;
    return MK_OK;
}

// Co-residency check, then the launch of `fn` (a persistent kernel over
// `workers` workgroups).
// Orders a launch on `stream` after the device's previous launch (the
// caller holds st->launch_mutex): same stream, nothing to do; another
// stream waits on an event recorded on the previous one now, which follows
// all the work queued there.  If that stream no longer exists (recording
// fails), its work has been handed to the device already, and a device
// synchronisation covers it.
int order_after_previous(DeviceState *st, hipStream_t stream, bool may_allocate) {
    if (!st->launched || st->last_stream == stream) return MK_OK;
    // the no-allocation launch records and waits on nothing (its callers may
    // be capturing a graph, where a wait on another stream's event is not
    // allowed): its caller orders it after launches on other streams
    if (!may_allocate) return MK_OK;
    hipError_t e;
    if (st->order_event == nullptr &&
        (e = hipEventCreateWithFlags(&st->order_event, hipEventDisableTiming)) != hipSuccess)
        return hip_fail(e, "hipEventCreateWithFlags");
    e = hipEventRecord(st->order_event, st->last_stream);
    if (e == hipSuccess) {
        e = hipStreamWaitEvent(stream, st->order_event, 0);
        if (e != hipSuccess) return hip_fail(e, "hipStreamWaitEvent");
        return MK_OK;
    }
    (void)hipGetLastError();
    if ((e = hipDeviceSynchronize()) != hipSuccess) return hip_fail(e, "hipDeviceSynchronize");
    return MK_OK;
}

// Co-residency check, ordering after the device's previous launch, then the
// launch of `fn` (a persistent kernel over `workers` workgroups).  The
// caller holds st->launch_mutex.
int launch_persistent(const void *fn, DeviceState *st, int64_t workers, size_t lds, KParams &kp,
                      hipStream_t stream, bool may_allocate = true) {
    int blocks = 0;
    hipError_t e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&blocks, fn, kThreads, lds);
    if (e != hipSuccess) return hip_fail(e, "hipOccupancyMaxActiveBlocksPerMultiprocessor");
    if (workers > (int64_t)blocks * st->num_cus) return MK_ERR_NOT_CORESIDENT;
    const int rc = order_after_previous(st, stream, may_allocate);
    if (rc != MK_OK) return rc;
    void *args[] = {&kp};
    e = hipLaunchKernel(fn, dim3((unsigned)workers), dim3(kThreads), args, lds, stream);
    if (e != hipSuccess) return hip_fail(e, "hipLaunchKernel");
    e = hipGetLastError();
    if (e != hipSuccess) return hip_fail(e, "hipGetLastError");
    // a no-allocation launch is ordered by its caller and is not what a later
    // launch orders itself after: its stream may be capturing a graph, and
    // an event recorded there for a launch on another stream would pull
    // that stream into the capture
    if (may_allocate) {
        st->launched = true;
        st->last_stream = stream;
    }
    return MK_OK;
}

// Spread-counter layout of a launch (scratch ints): the parts follow the
// cursors and column-chunk counters, kSpreadAlign-aligned.  MK_SPREAD=0 in
// the environment turns them off (a measurement switch: every arrival then
// goes to the barrier tensor itself).
struct SpreadLayout {
    bool on;
    int32_t ops;
    size_t offset, rows, stride, end;
};

// Launch-time tuning overrides, for measurements: MK_SPREAD, MK_SPIN_SLEEP,
// MK_TAIL, MK_EARLY, MK_PF, MK_STAGE_ITEMS and MK_CODE_PF.  The environment is read once
// per process, at the first launch (mk_mixtral_reload_overrides reads it
// again).  A value that is not a whole number is ignored with a warning on
// stderr, and each override in effect is reported there when it is read, so
// a stray variable in a serving process shows instead of silently changing
// the scheduling.
enum { kOvSpread, kOvSpinSleep, kOvTail, kOvEarly, kOvPf, kOvStageItems, kOvCodePf, kOvCount };
struct TuningOverride {
    const char *name;
    bool set;
    long value;
};
TuningOverride g_overrides[kOvCount] = {{"MK_SPREAD", false, 0}, {"MK_SPIN_SLEEP", false, 0},
                                        {"MK_TAIL", false, 0},   {"MK_EARLY", false, 0},
                                        {"MK_PF", false, 0},     {"MK_STAGE_ITEMS", false, 0},
                                        {"MK_CODE_PF", false, 0}};
std::mutex g_overrides_mutex;
bool g_overrides_read = false;

void read_overrides_locked() {
    for (TuningOverride &o : g_overrides) {
        o.set = false;
        const char *env = std::getenv(o.name);
        if (env == nullptr || *env == '\0') continue;
        char *end = nullptr;
        errno = 0;
        const long v = std::strtol(env, &end, 0);
        while (end != nullptr && std::isspace((unsigned char)*end)) ++end;
        if (errno != 0 || end == env || end == nullptr || *end != '\0') {
            std::fprintf(stderr, "mk_mixtral: ignoring %s=\"%s\" (not a whole number)\n", o.name, env);
            continue;
        }
        o.set = true;
        o.value = v;
        std::fprintf(stderr, "mk_mixtral: measurement override %s=%ld in effect\n", o.name, v);
    }
    g_overrides_read = true;
}

// The override `k`, or nothing: `*value` is set only when one is in effect.
bool tuning_override(int k, long *value) {
    std::lock_guard<std::mutex> lock(g_overrides_mutex);
    if (!g_overrides_read) read_overrides_locked();
    if (!g_overrides[k].set) return false;
    *value = g_overrides[k].value;
    return true;
}

// `ops`: bit k set spreads the counters of opcode k (the default is the
// caller's); MK_SPREAD=<bits> overrides it for measurements.
SpreadLayout spread_layout(size_t used, int64_t layers, int64_t bar_ops, int32_t ops) {
    SpreadLayout s{};
    long v = 0;
    if (tuning_override(kOvSpread, &v)) ops = (int32_t)v;
    s.ops = ops;
    s.on = ops != 0;
    s.rows = (size_t)layers * (size_t)bar_ops;
    s.stride = (s.rows + kSpreadAlign - 1) / kSpreadAlign * kSpreadAlign;
    s.offset = (used + kSpreadAlign - 1) / kSpreadAlign * kSpreadAlign;
    s.end = s.on ? s.offset + (size_t)kSpread * s.stride : used;
    return s;
}

// A tuning value of the launch: `def`, or the override `k` (for
// measurements), clamped to [lo, hi].
int32_t tuning_value(int k, long def, long lo, long hi) {
    long v = def;
    (void)tuning_override(k, &v);
    return (int32_t)std::min(hi, std::max(lo, v));
}

// Longest spin back-off (MK_SPIN_SLEEP_MAX naps, MK_SPIN_SLEEP overrides it).
int32_t spin_max_naps() { return tuning_value(kOvSpinSleep, MK_SPIN_SLEEP_MAX, 1, 64); }

// Opcode-5 items staged ahead in LDS: `n` (what the LDS holds), none with
// late loads; MK_STAGE_ITEMS=<k> caps it for measurements.
size_t stage_limit(size_t n, bool late_loads) {
    long v = 0;
    if (tuning_override(kOvStageItems, &v)) n = std::min(n, (size_t)std::max(0L, v));
    return late_loads ? 0 : n;
}

// Machine-code bytes code_prefetch reads for a kernel whose measured length
// is `len` (0 in a library compiled without the measurement); MK_CODE_PF=0
// turns the prefetch off for measurements.
uint32_t code_prefetch_len(uint32_t len) {
    long v = 1;
    (void)tuning_override(kOvCodePf, &v);
    return v != 0 ? len : 0u;
}

uint32_t timeout_ticks(uint32_t spin_timeout_us) {
    const uint64_t us = spin_timeout_us ? spin_timeout_us : 2000000u;
    const uint64_t ticks = us * kTicksPerUs;
    return ticks > 0xffffffffu ? 0xffffffffu : (uint32_t)ticks;
}

// ceil(2^32 / d) for d >= 2: spread_row's exact division of n < 2^16 by d < 2^16.
uint32_t div_magic(int32_t d) { return d >= 2 ? (uint32_t)(((1ull << 32) + (uint64_t)d - 1) / (uint64_t)d) : 0u; }

// Divisors of spread_row; spreading stays off where they would not be exact.
void set_spread_divisors(KParams &kp, int64_t layers) {
    const int64_t ints = layers * (int64_t)kp.bar_ops * (int64_t)kp.bar_width;
    kp.bar_width_magic = div_magic(kp.bar_width);
    kp.bar_ops_magic = div_magic(kp.bar_ops);
    kp.bar_ints = (int32_t)std::min<int64_t>(ints, 1 << 16);
    if (ints >= (1 << 16) || kp.bar_width < 2 || kp.bar_ops < 2) kp.spread = nullptr;
}

// Dynamic LDS for the launch with an opcode-2 ring of `kv_ring` chunks
// (ignored without attention tensors).
size_t lds_bytes_for(const mk_mixtral_globals *g, int kv_ring) {
    const size_t normed = (size_t)g->hidden_size * 2;
    // both SiLU rows, then the opcode-6 cache-warming sink (1 KiB per wave)
    const size_t silu = (size_t)g->intermediate_size * 2 * 2 + (size_t)kWaves * 1024;
    size_t need = normed > silu ? normed : silu;
    if (g->qkv_weights != nullptr) {
        const size_t Hq = (size_t)g->num_attention_heads, Hkv = (size_t)g->num_kv_heads, D = (size_t)g->head_dim;
        // opcode 1: normed hidden + one fp32 per QKV row; opcode 2: the K/V
        // ring, then per-wave softmax partials; opcode 4: attn_out
        const size_t qkv = normed + (Hq + 2 * Hkv) * D * 4;
        const size_t attn = (size_t)kv_ring * kKvChunkBytes + (size_t)kWaves * (Hq / Hkv) * (D + 2) * 4;
        const size_t oproj = Hq * D * 2;
        need = need > qkv ? need : qkv;
        need = need > attn ? need : attn;
        need = need > oproj ? need : oproj;
    }
    return need > (size_t)kMinLdsBytes ? need : (size_t)kMinLdsBytes;
}

// Largest opcode-2 ring (chunks: kKvRingMax or kAttnSub) whose launch fits
// in `max_lds` bytes of LDS per workgroup; 0 if neither does.
int kv_ring_for(const mk_mixtral_globals *g, size_t max_lds) {
    // whole groups of kAttnSub chunks (opcode 2 computes a group at a time)
    for (int nb = kKvRingMax; nb >= kAttnSub; nb -= kAttnSub)
        if (lds_bytes_for(g, nb) + sizeof(SharedState) <= max_lds) return nb;
    return 0;
}

// The attention tensors are optional (an MoE-only launch passes none); when
// qkv_weights is set, every attention field must be consistent.
int validate_attention(const mk_mixtral_globals *g) {
    if (g->qkv_weights == nullptr) return MK_OK;
    if (!g->attn_norm_weights || !g->o_weights || !g->lm_head_norm_weights || !g->lm_head_weights || !g->k_cache ||
        !g->v_cache || !g->rope_cos || !g->rope_sin || !g->q_post_rope || !g->attn_out ||
        !g->attn_lse_intermediates || !g->attn_out_intermediates || !g->logits)
        return MK_ERR_INVALID_ARGUMENT;
    const int Hq = g->num_attention_heads, Hkv = g->num_kv_heads, D = g->head_dim;
    if (Hkv < 1 || Hq < Hkv || Hq % Hkv || Hq / Hkv > 4) return MK_ERR_UNSUPPORTED;
    if (D != 64 && D != 128) return MK_ERR_UNSUPPORTED;
    if ((Hq * D) % kChunkElems) return MK_ERR_UNSUPPORTED;
    if (g->qkv_block_size < 2 || g->qkv_block_size % 2 || D % g->qkv_block_size) return MK_ERR_INVALID_ARGUMENT;
    if (g->o_proj_block_size % 2 || g->lm_head_block_size < 2 || g->lm_head_block_size % 2) return MK_ERR_INVALID_ARGUMENT;
    if (g->attn_kv_block_size < 1 || g->vocab_size < 1 || g->vocab_size % g->lm_head_block_size)
        return MK_ERR_INVALID_ARGUMENT;
    if (g->lm_head_reduction < kChunkElems || g->lm_head_reduction % kChunkElems) return MK_ERR_INVALID_ARGUMENT;
    if (g->kv_capacity < 1 || (int64_t)g->pos_id >= g->kv_capacity || g->attn_partial_slots < 1)
        return MK_ERR_INVALID_ARGUMENT;
    // KV slabs are addressed with 32-bit byte offsets per layer
    if ((int64_t)g->kv_capacity * Hkv * D * 2 > (INT64_C(1) << 31) - 1) return MK_ERR_UNSUPPORTED;
    if (!aligned16(g->qkv_weights) || !aligned16(g->o_weights) || !aligned16(g->lm_head_weights) ||
        !aligned16(g->k_cache) || !aligned16(g->v_cache) || !aligned16(g->q_post_rope) || !aligned16(g->attn_out) ||
        !aligned16(g->attn_norm_weights) || !aligned16(g->lm_head_norm_weights) ||
        (reinterpret_cast<uintptr_t>(g->logits) & 3u))
        return MK_ERR_INVALID_ARGUMENT;
    return MK_OK;
}

int validate(const mk_mixtral_globals *g) {
    if (g == nullptr || g->struct_size < sizeof(mk_mixtral_globals) || g->abi_version != MK_MIXTRAL_ABI_VERSION)
        return MK_ERR_INVALID_ARGUMENT;
    if (!g->barriers || !g->instructions || !g->expert_gate_weights || !g->expert_up_weights ||
        !g->expert_down_weights || !g->router_weights || !g->ffn_ln_weights || !g->hidden_states ||
        !g->expert_silu_out || !g->router_normed_hidden || !g->selected_expert_indices ||
        !g->selected_expert_scores || !g->predicted_expert_indices)
        return MK_ERR_INVALID_ARGUMENT;
    if (g->num_workers < 1 || g->queue_len < 1 || g->num_workers > (1 << 20) || g->queue_len > (1 << 20))
        return MK_ERR_INVALID_ARGUMENT;
    if (g->num_layers < 1 || g->bar_layers < g->num_layers || g->bar_ops < 8 || g->bar_width < 1)
        return MK_ERR_INVALID_ARGUMENT;
    if (g->num_experts_per_tok != 2 || g->num_experts < 2 || g->num_experts > MK_MAX_EXPERTS)
        return MK_ERR_UNSUPPORTED;
    if (g->hidden_size < kChunkElems || g->hidden_size % kChunkElems || g->intermediate_size < kChunkElems ||
        g->intermediate_size % kChunkElems || g->intermediate_size > kMaxIntermediate)
        return MK_ERR_UNSUPPORTED;
    if (g->expert_proj_block_size < 1 || g->down_proj_block_size < 1 || g->o_proj_block_size < 1 ||
        g->intermediate_size % g->expert_proj_block_size || g->hidden_size % g->down_proj_block_size ||
        g->hidden_size % g->o_proj_block_size)
        return MK_ERR_INVALID_ARGUMENT;
    if ((int64_t)g->num_layers * g->num_experts * g->intermediate_size * (int64_t)g->hidden_size > (INT64_C(1) << 40))
        return MK_ERR_UNSUPPORTED;
    if (!(g->rms_norm_eps >= 0.0f) || !isfinite(g->rms_norm_eps)) return MK_ERR_INVALID_ARGUMENT;
    const void *vec[] = {g->expert_gate_weights, g->expert_up_weights, g->expert_down_weights, g->router_weights,
                         g->ffn_ln_weights,      g->hidden_states,     g->expert_silu_out,     g->router_normed_hidden,
                         g->predictor_weights};
    for (const void *v : vec)
        if (v != nullptr && !aligned16(v)) return MK_ERR_INVALID_ARGUMENT;
    if (g->next_embed_weights != nullptr && (g->argmax_out == nullptr || !aligned16(g->next_embed_weights)))
        return MK_ERR_INVALID_ARGUMENT;
    if (g->argmax_out != nullptr &&
        (g->qkv_weights == nullptr || g->logits == nullptr || (reinterpret_cast<uintptr_t>(g->argmax_out) & 7u)))
        return MK_ERR_INVALID_ARGUMENT;
    return validate_attention(g);
}

// ---- dense Llama launches ----

size_t lds_bytes_llama(const mk_llama_globals *g, int kv_ring) {
    const size_t H = (size_t)g->hidden_size, Hq = (size_t)g->num_attention_heads,
                 Hkv = (size_t)g->num_kv_heads, D = (size_t)g->head_dim;
    size_t need = H * 2;                                         // normed hidden (opcodes 5, 7)
    const size_t qkv = H * 2 + (Hq + 2 * Hkv) * D * 4;           // opcode 1
    const size_t attn = (size_t)kv_ring * kKvChunkBytes + (size_t)kWaves * (Hq / Hkv) * (D + 2) * 4;  // opcode 2
    const size_t oproj = Hq * D * 2;                             // opcode 4
    const size_t down = (size_t)g->matvec_reduction_size * 2;    // opcode 6
    for (size_t v : {qkv, attn, oproj, down}) need = need > v ? need : v;
    return need > (size_t)kMinLdsBytes ? need : (size_t)kMinLdsBytes;
}

int kv_ring_llama(const mk_llama_globals *g, size_t max_lds) {
    for (int nb = kKvRingMax; nb >= kAttnSub; nb -= kAttnSub)
        if (lds_bytes_llama(g, nb) + sizeof(SharedState) <= max_lds) return nb;
    return 0;
}

int validate_llama(const mk_llama_globals *g) {
    if (g == nullptr || g->struct_size < sizeof(mk_llama_globals) || g->abi_version != MK_LLAMA_ABI_VERSION)
        return MK_ERR_INVALID_ARGUMENT;
    if (!g->barriers || !g->instructions || !g->qkv_weights || !g->attn_norm_weights || !g->o_weights ||
        !g->mlp_norm_weights || !g->up_weights || !g->gate_weights || !g->down_weights ||
        !g->lm_head_norm_weights || !g->lm_head_weights || !g->k_cache || !g->v_cache || !g->rope_cos ||
        !g->rope_sin || !g->hidden_states || !g->q_post_rope || !g->attn_out || !g->attn_lse_intermediates ||
        !g->attn_out_intermediates || !g->silu_out || !g->logits)
        return MK_ERR_INVALID_ARGUMENT;
    if (g->num_workers < 1 || g->queue_len < 1 || g->num_workers > (1 << 20) || g->queue_len > (1 << 20))
        return MK_ERR_INVALID_ARGUMENT;
    if (g->num_layers < 1 || g->bar_layers < g->num_layers || g->bar_ops < 7 || g->bar_width < 1)
        return MK_ERR_INVALID_ARGUMENT;
    const int H = g->hidden_size, F = g->intermediate_size, Hq = g->num_attention_heads, Hkv = g->num_kv_heads,
              D = g->head_dim;
    if (H < kChunkElems || H % kChunkElems || F < 2 || (int64_t)F * H > (INT64_C(1) << 40)) return MK_ERR_UNSUPPORTED;
    if (Hkv < 1 || Hq < Hkv || Hq % Hkv || Hq / Hkv > 4) return MK_ERR_UNSUPPORTED;
    if (D != 64 && D != 128) return MK_ERR_UNSUPPORTED;
    if ((Hq * D) % kChunkElems) return MK_ERR_UNSUPPORTED;
    if (g->bar_width < Hq + 2 * Hkv) return MK_ERR_INVALID_ARGUMENT;
    const int R = g->matvec_reduction_size;
    if (R < kChunkElems || R % kChunkElems || F % R) return MK_ERR_UNSUPPORTED;
    // opcode 6 takes full rows when R == F, else items of 16 / (R / 512)
    // rows x R / 512 chunks
    const int rc = R / kChunkElems;
    if (R != F && rc != 1 && rc != 2 && rc != 4 && rc != 8) return MK_ERR_UNSUPPORTED;
    if (R != F && g->down_proj_block_size % (16 / rc)) return MK_ERR_UNSUPPORTED;
    if (g->up_gate_proj_block_size < 1 || F % g->up_gate_proj_block_size || g->down_proj_block_size < 2 ||
        g->down_proj_block_size % 2 || H % g->down_proj_block_size || g->o_proj_block_size < 2 ||
        g->o_proj_block_size % 2 || H % g->o_proj_block_size)
        return MK_ERR_INVALID_ARGUMENT;
    if (g->qkv_block_size < 2 || g->qkv_block_size % 2 || D % g->qkv_block_size) return MK_ERR_INVALID_ARGUMENT;
    if (g->lm_head_block_size < 2 || g->lm_head_block_size % 2 || g->vocab_size < 1 ||
        g->vocab_size % g->lm_head_block_size || g->attn_kv_block_size < 1)
        return MK_ERR_INVALID_ARGUMENT;
    if (g->kv_capacity < 1 || (int64_t)g->pos_id >= g->kv_capacity || g->attn_partial_slots < 1)
        return MK_ERR_INVALID_ARGUMENT;
    if ((int64_t)g->kv_capacity * Hkv * D * 2 > (INT64_C(1) << 31) - 1) return MK_ERR_UNSUPPORTED;
    if (!(g->rms_norm_eps >= 0.0f) || !isfinite(g->rms_norm_eps)) return MK_ERR_INVALID_ARGUMENT;
    const void *vec[] = {g->qkv_weights, g->attn_norm_weights, g->o_weights, g->mlp_norm_weights, g->up_weights,
                         g->gate_weights, g->down_weights, g->lm_head_norm_weights, g->lm_head_weights, g->k_cache,
                         g->v_cache, g->hidden_states, g->q_post_rope, g->attn_out, g->silu_out};
    for (const void *v : vec)
        if (!aligned16(v)) return MK_ERR_INVALID_ARGUMENT;
    if (reinterpret_cast<uintptr_t>(g->logits) & 3u) return MK_ERR_INVALID_ARGUMENT;
    if (g->next_embed_weights != nullptr && (g->argmax_out == nullptr || !aligned16(g->next_embed_weights)))
        return MK_ERR_INVALID_ARGUMENT;
    if (g->argmax_out != nullptr && (reinterpret_cast<uintptr_t>(g->argmax_out) & 7u)) return MK_ERR_INVALID_ARGUMENT;
    return MK_OK;
}

}  // namespace

extern "C" {

int mk_llama_abi_version(void) { return MK_LLAMA_ABI_VERSION; }

int mk_llama_launch(const mk_llama_globals *g, void *stream) {
    int rc = validate_llama(g);
    if (rc != MK_OK) return rc;
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return hip_fail(e, "hipGetDevice");
    DeviceState *st = nullptr;
    rc = device_state(dev, &st);
    if (rc != MK_OK) return rc;
    std::lock_guard<std::mutex> launch_lock(st->launch_mutex);
    const int kv_ring = kv_ring_llama(g, (size_t)st->max_lds);
    if (kv_ring < 1) return MK_ERR_UNSUPPORTED;
    size_t lds = lds_bytes_llama(g, kv_ring);
    // opcode-5 staging area: after the O-proj input and the normed hidden
    // state (both at offset 0), up to the LDS a workgroup may have
    const size_t at0 = std::max((size_t)g->hidden_size, (size_t)g->num_attention_heads * g->head_dim);
    const size_t stage_off = ((at0 * 2 + 1023) / 1024) * 1024;
    const size_t stage_item = (size_t)g->hidden_size * 4;
    const size_t lds_cap = (size_t)st->max_lds - sizeof(SharedState);
    const size_t stage_items = stage_limit(
        lds_cap > stage_off ? std::min((size_t)MK_STAGE_ITEMS, (lds_cap - stage_off) / stage_item) : 0, g->late_loads);
    if (stage_items > 0) lds = std::max(lds, stage_off + stage_items * stage_item);
    // scratch: the work-claim slots, then the exit argmax's candidates (2
    // ints per workgroup), then the spread counters
    const size_t cand = kScratchSlotBase + 2 * (size_t)g->num_workers * (size_t)g->queue_len;
    const SpreadLayout sp = spread_layout(cand + 2 * (size_t)g->num_workers, g->num_layers, g->bar_ops,
                                          kSpreadDenseOps);
    rc = ensure_scratch(st, sp.end);
    if (rc != MK_OK) return rc;

    KParams kp{};
    kp.chunk_ctr = nullptr;
    kp.lm_cand = g->argmax_out != nullptr ? st->scratch + cand : nullptr;
    kp.spread = sp.on ? st->scratch + sp.offset : nullptr;
    kp.spread_rows = (int32_t)sp.rows;
    kp.spread_stride = (int32_t)sp.stride;
    kp.spread_ops = sp.ops;
    // the last workgroup zeroes the claim slots and the candidates (after
    // the exit argmax has read them): every launch starts from zeroed scratch
    kp.scratch_clear = (int32_t)(cand + 2 * (size_t)g->num_workers - kScratchSlotBase);
    kp.instructions = g->instructions;
    kp.timings = g->record_timings ? g->timings : nullptr;
    kp.bar = g->barriers;
    kp.status = g->status != nullptr ? g->status : st->status;
    // the dense MLP is the one-expert case of the MoE weight layout
    kp.gate = g->gate_weights;
    kp.up = g->up_weights;
    kp.down = g->down_weights;
    kp.ffn_ln = g->mlp_norm_weights;
    kp.hidden = g->hidden_states;
    kp.silu = g->silu_out;
    kp.queue_len = (int32_t)g->queue_len;
    kp.num_layers = g->num_layers;
    kp.H = g->hidden_size;
    kp.F = g->intermediate_size;
    kp.E = 1;
    kp.bar_ops = (int32_t)g->bar_ops;
    kp.bar_width = (int32_t)g->bar_width;
    set_spread_divisors(kp, g->num_layers);
    kp.expert_bs = g->up_gate_proj_block_size;
    kp.down_bs = g->down_proj_block_size;
    kp.oproj_bs = g->o_proj_block_size;
    kp.eps = g->rms_norm_eps;
    kp.timeout_ticks = timeout_ticks(g->spin_timeout_us);
    kp.scratch = st->scratch;
    kp.work_sharing = 0;
    kp.spin_max = spin_max_naps();
    kp.tail_items = tuning_value(kOvTail, MK_TAIL_ITEMS, 1, 1 << 20);
    kp.early_loads = tuning_value(kOvEarly, MK_EARLY_LOADS, 0, 1);
    kp.pf_rounds = tuning_value(kOvPf, MK_PF_ROUNDS, 0, 4);
    kp.ostage = 0;
    kp.code_len = code_prefetch_len(MK_CODE_LEN_LLAMA);
    kp.red_cols = g->matvec_reduction_size;
    kp.late_loads = g->late_loads ? 1 : 0;
    kp.stage_items = (int32_t)stage_items;
    kp.stage_off16 = (int32_t)(stage_off / 16);
    kp.lds_bytes = (int32_t)lds;
    kp.down_arrivals = (g->intermediate_size / g->matvec_reduction_size) * (g->hidden_size / g->down_proj_block_size);
    kp.argmax_out = g->argmax_out;
    kp.next_embed = g->next_embed_weights;
    kp.reset_next = g->reset_for_next_launch ? 1 : 0;
    kp.attn = 1;
    AttnParams a{};
    a.qkv = g->qkv_weights;
    a.attn_ln = g->attn_norm_weights;
    a.oproj = g->o_weights;
    a.lm_norm = g->lm_head_norm_weights;
    a.lm_head = g->lm_head_weights;
    a.kc = g->k_cache;
    a.vc = g->v_cache;
    a.q_rope = g->q_post_rope;
    a.attn_out = g->attn_out;
    a.logits = g->logits;
    a.rope_cos = g->rope_cos;
    a.rope_sin = g->rope_sin;
    a.lse_int = g->attn_lse_intermediates;
    a.out_int = g->attn_out_intermediates;
    a.Hq = g->num_attention_heads;
    a.Hkv = g->num_kv_heads;
    a.D = g->head_dim;
    a.V = g->vocab_size;
    a.T = g->kv_capacity;
    a.P = g->attn_partial_slots;
    a.qkv_bs = g->qkv_block_size;
    a.kv_bs = g->attn_kv_block_size;
    a.lm_bs = g->lm_head_block_size;
    a.lm_red = g->hidden_size;
    a.attn_scale = g->attn_scale;
    a.skip_red = g->skip_attn_reduction ? 1 : 0;
    a.kv_ring = kv_ring;
    kp.attn_params = a;
    kp.pos = g->pos_id;
    return launch_persistent(reinterpret_cast<const void *>(mk_llama_kernel), st, g->num_workers, lds, kp,
                             reinterpret_cast<hipStream_t>(stream));
}

int mk_mixtral_abi_version(void) { return MK_MIXTRAL_ABI_VERSION; }

void mk_mixtral_reload_overrides(void) {
    std::lock_guard<std::mutex> lock(g_overrides_mutex);
    read_overrides_locked();
}

int mk_mixtral_last_hip_error(void) { return g_last_hip_error; }

const char *mk_mixtral_last_error_site(void) { return g_last_hip_site; }

const char *mk_mixtral_error_string(int code) {
    switch (code) {
    case MK_OK: return "ok";
    case MK_ERR_INVALID_ARGUMENT: return "invalid argument";
    case MK_ERR_UNSUPPORTED: return "shape or configuration not supported by the kernel";
    case MK_ERR_HIP: return "HIP runtime error";
    case MK_ERR_NOT_CORESIDENT: return "worker count exceeds co-resident workgroups";
    case MK_ERR_SCRATCH_TOO_SMALL:
        return "the launch needs more scratch than mk_mixtral_launch_noalloc's fixed 2 MiB array holds "
               "(fewer workers x queue slots)";
    case MK_ERR_TIMEOUT: return "barrier wait timed out";
    case MK_ERR_BAD_OPCODE: return "unknown opcode";
    case MK_ERR_UNSUPPORTED_OPCODE: return "opcode not implemented by this kernel (attention / LM head)";
    case MK_ERR_BAD_INSTRUCTION: return "instruction operand out of range";
    default: return "unknown status code";
    }
}

int mk_mixtral_query_device(int device, int32_t *num_cus, int32_t *max_workers) {
    DeviceGuard guard(device);
    if (guard.err != hipSuccess) return hip_fail(guard.err, "hipSetDevice");
    DeviceState *st = nullptr;
    int rc = device_state(device, &st);
    if (rc != MK_OK) return rc;
    int blocks = 0;
    hipError_t e = hipOccupancyMaxActiveBlocksPerMultiprocessor(
        &blocks, reinterpret_cast<const void *>(mk_mixtral_kernel<0, true>), kThreads, kMinLdsBytes);
    if (e != hipSuccess) return hip_fail(e, "hipOccupancyMaxActiveBlocksPerMultiprocessor");
    if (num_cus) *num_cus = st->num_cus;
    if (max_workers) *max_workers = blocks * st->num_cus;
    return MK_OK;
}

// mk_mixtral_launch and mk_mixtral_launch_noalloc: `noalloc` takes the
// launch's scratch from the fixed device array (and its status words there
// too when the caller passes none) and allocates nothing.
static int launch_mixtral(const mk_mixtral_globals *g, void *stream, bool noalloc) {
    int rc = validate(g);
    if (rc != MK_OK) return rc;
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return hip_fail(e, "hipGetDevice");
    DeviceState *st = nullptr;
    rc = device_state(dev, &st, !noalloc, noalloc);
    if (rc != MK_OK) return rc;
    std::lock_guard<std::mutex> launch_lock(st->launch_mutex);

    const int kv_ring = kv_ring_for(g, (size_t)st->max_lds);
    if (kv_ring < 1) return MK_ERR_UNSUPPORTED;
    const size_t lds = lds_bytes_for(g, kv_ring);
    // Mixtral's 8 experts get a kernel specialised for exactly 8
    const bool e8 = g->num_experts == 8;
    const bool attn = g->qkv_weights != nullptr;
    const void *fn = e8 ? (attn ? reinterpret_cast<const void *>(mk_mixtral_kernel<8, true>)
                                : reinterpret_cast<const void *>(mk_mixtral_kernel<8, false>))
                        : (attn ? reinterpret_cast<const void *>(mk_mixtral_kernel<0, true>)
                                : reinterpret_cast<const void *>(mk_mixtral_kernel<0, false>));
    // scratch: exit counter, work-sharing cursors, then (overlap on) the
    // column-chunk counters of every layer
    const size_t cursors = 2 * (size_t)g->num_workers * (size_t)g->queue_len;
    // compiled into the 8-expert MoE-only kernel only
    const bool overlap = g->downproj_overlap != 0 && !g->work_sharing && g->num_experts == 8 &&
                         g->qkv_weights == nullptr;
    const size_t chunks = overlap ? (size_t)g->num_layers * (size_t)(g->intermediate_size / 512) : 0;
    const SpreadLayout sp = spread_layout(kScratchSlotBase + cursors + chunks, g->num_layers, g->bar_ops,
                                          attn ? kSpreadMixtralOps : kSpreadMoeOps);
    int32_t *base = nullptr;
    if (noalloc) {
        if (sp.end > kNoAllocScratchInts - kNoAllocBaseInts) return MK_ERR_SCRATCH_TOO_SMALL;
        base = st->noalloc_scratch + kNoAllocBaseInts;
    } else {
        rc = ensure_scratch(st, sp.end);
        if (rc != MK_OK) return rc;
        base = st->scratch;
    }

    KParams kp{};  // every field the launch does not set is zero (null lm_cand: the exit argmax reads the logits)
    kp.chunk_ctr = overlap ? base + kScratchSlotBase + cursors : nullptr;
    kp.spread = sp.on ? base + sp.offset : nullptr;
    kp.spread_rows = (int32_t)sp.rows;
    kp.spread_stride = (int32_t)sp.stride;
    kp.spread_ops = sp.ops;
    kp.scratch_clear = (int32_t)(cursors + chunks);
    kp.instructions = g->instructions;
    kp.timings = g->record_timings ? g->timings : nullptr;
    kp.bar = g->barriers;
    kp.status = g->status != nullptr ? g->status : noalloc ? st->noalloc_scratch : st->status;
    kp.gate = g->expert_gate_weights;
    kp.up = g->expert_up_weights;
    kp.down = g->expert_down_weights;
    kp.router = g->router_weights;
    kp.predictor = g->predictor_weights;
    kp.ffn_ln = g->ffn_ln_weights;
    kp.router_bias = g->router_bias;
    kp.hidden = g->hidden_states;
    kp.silu = g->expert_silu_out;
    kp.normed_out = g->router_normed_hidden;
    kp.sel_idx = g->selected_expert_indices;
    kp.sel_score = g->selected_expert_scores;
    kp.pred_idx = g->predicted_expert_indices;
    kp.queue_len = (int32_t)g->queue_len;
    kp.num_layers = g->num_layers;
    kp.H = g->hidden_size;
    kp.F = g->intermediate_size;
    kp.E = g->num_experts;
    kp.bar_ops = (int32_t)g->bar_ops;
    kp.bar_width = (int32_t)g->bar_width;
    set_spread_divisors(kp, g->num_layers);
    kp.expert_bs = g->expert_proj_block_size;
    kp.down_bs = g->down_proj_block_size;
    kp.oproj_bs = g->o_proj_block_size;
    kp.eps = g->rms_norm_eps;
    kp.timeout_ticks = timeout_ticks(g->spin_timeout_us);
    kp.scratch = base;
    kp.work_sharing = g->work_sharing ? 1 : 0;
    kp.spin_max = spin_max_naps();
    kp.tail_items = tuning_value(kOvTail, MK_TAIL_ITEMS, 1, 1 << 20);
    kp.early_loads = tuning_value(kOvEarly, MK_EARLY_LOADS, 0, 1);
    kp.pf_rounds = tuning_value(kOvPf, MK_PF_ROUNDS, 0, 4);
    kp.ostage = 1;
    kp.code_len = code_prefetch_len(e8 ? (attn ? MK_CODE_LEN_E8_ATTN : MK_CODE_LEN_E8)
                                         : (attn ? MK_CODE_LEN_E0_ATTN : MK_CODE_LEN_E0));
    kp.down_arrivals = 2 * (g->hidden_size / g->down_proj_block_size);
    kp.red_cols = 0;
    // whole-model launches: the O projection stages up to one predicted
    // opcode-5 item per wave (but wave 0) in the LDS after its attention
    // vector (opcode 5's normed hidden state), within the launch's LDS (the
    // opcode-2 ring makes it ~145 KiB at the Mixtral shape)
    const size_t at0 = attn ? std::max((size_t)g->hidden_size, (size_t)g->num_attention_heads * g->head_dim)
                            : (size_t)g->hidden_size;
    const size_t stage_off = ((at0 * 2 + 1023) / 1024) * 1024;
    const size_t stage_item = (size_t)g->hidden_size * 4;
    kp.late_loads = g->late_loads ? 1 : 0;
    kp.stage_items = (int32_t)stage_limit(
        attn && lds > stage_off ? std::min((size_t)(kWaves - 1), (lds - stage_off) / stage_item) : 0, g->late_loads);
    kp.stage_off16 = (int32_t)(stage_off / 16);
    kp.lds_bytes = (int32_t)lds;
    kp.argmax_out = g->argmax_out;
    kp.next_embed = g->next_embed_weights;
    kp.reset_next = g->reset_for_next_launch ? (g->qkv_weights != nullptr ? 2 : 1) : 0;
    kp.attn = g->qkv_weights != nullptr;
    kp.attn_params = AttnParams{};
    if (kp.attn) {
        AttnParams a{};
        a.qkv = g->qkv_weights;
        a.attn_ln = g->attn_norm_weights;
        a.oproj = g->o_weights;
        a.lm_norm = g->lm_head_norm_weights;
        a.lm_head = g->lm_head_weights;
        a.kc = g->k_cache;
        a.vc = g->v_cache;
        a.q_rope = g->q_post_rope;
        a.attn_out = g->attn_out;
        a.logits = g->logits;
        a.rope_cos = g->rope_cos;
        a.rope_sin = g->rope_sin;
        a.lse_int = g->attn_lse_intermediates;
        a.out_int = g->attn_out_intermediates;
        a.Hq = g->num_attention_heads;
        a.Hkv = g->num_kv_heads;
        a.D = g->head_dim;
        a.V = g->vocab_size;
        a.T = g->kv_capacity;
        a.P = g->attn_partial_slots;
        a.qkv_bs = g->qkv_block_size;
        a.kv_bs = g->attn_kv_block_size;
        a.lm_bs = g->lm_head_block_size;
        a.lm_red = g->lm_head_reduction;
        a.attn_scale = g->attn_scale;
        a.skip_red = g->skip_attn_reduction ? 1 : 0;
        a.kv_ring = kv_ring;
        kp.attn_params = a;
    }
    kp.pos = g->pos_id;
    // fn is one of the four instantiations above
    return launch_persistent(fn, st, g->num_workers, lds, kp, reinterpret_cast<hipStream_t>(stream), !noalloc);
}

int mk_mixtral_launch(const mk_mixtral_globals *g, void *stream) { return launch_mixtral(g, stream, false); }

int mk_mixtral_launch_noalloc(const mk_mixtral_globals *g, void *stream) { return launch_mixtral(g, stream, true); }

int mk_mixtral_read_status(int device, int32_t *out) {
    if (out == nullptr) return MK_ERR_INVALID_ARGUMENT;
    DeviceGuard guard(device);
    if (guard.err != hipSuccess) return hip_fail(guard.err, "hipSetDevice");
    DeviceState *st = nullptr;
    int rc = device_state(device, &st);
    if (rc != MK_OK) return rc;
    hipError_t e = hipDeviceSynchronize();
    if (e == hipSuccess) e = hipMemcpy(out, st->status, MK_STATUS_WORDS * sizeof(int32_t), hipMemcpyDeviceToHost);
    // no failure there: the status words of mk_mixtral_launch_noalloc
    if (e == hipSuccess && out[MK_STATUS_CODE] == MK_OK && st->noalloc_scratch != nullptr)
        e = hipMemcpy(out, st->noalloc_scratch, MK_STATUS_WORDS * sizeof(int32_t), hipMemcpyDeviceToHost);
    if (e != hipSuccess) return hip_fail(e, "hipMemcpy");
    return MK_OK;
}

int mk_mixtral_clear_status(int device) {
    DeviceGuard guard(device);
    if (guard.err != hipSuccess) return hip_fail(guard.err, "hipSetDevice");
    DeviceState *st = nullptr;
    int rc = device_state(device, &st);
    if (rc != MK_OK) return rc;
    hipError_t e = hipDeviceSynchronize();
    if (e == hipSuccess) e = hipMemset(st->status, 0, MK_STATUS_WORDS * sizeof(int32_t));
    if (e == hipSuccess && st->noalloc_scratch != nullptr)
        e = hipMemset(st->noalloc_scratch, 0, MK_STATUS_WORDS * sizeof(int32_t));
    if (e == hipSuccess) e = hipDeviceSynchronize();
    if (e != hipSuccess) return hip_fail(e, "hipDeviceSynchronize");
    return MK_OK;
}

}  // extern "C"
