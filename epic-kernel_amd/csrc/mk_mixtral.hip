// Persistent MoE decode megakernel for MI355X (gfx950, CDNA4).
//
// One workgroup per compute unit runs its instruction queue in order
// (instruction layout: megakernels/instructions.py:97-119).  Workers meet only
// through int32 counters in HBM: an arrival is an agent-scope release
// fetch-add, a wait is a bounded spin of relaxed agent-scope loads followed by
// one agent-scope acquire fence.  There is no loader/consumer/storer split as
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
// 8-element product uses v_dot2 (bf16 pairs, fp32 accumulate); the row sum
// is a 64-lane butterfly.

#include <hip/hip_runtime.h>

#include <math.h>
#include <mutex>
#include <stddef.h>
#include <stdint.h>

#include "mk_mixtral.h"

#ifndef MK_THREADS
#define MK_THREADS 1024
#endif
#ifndef MK_NT_LOADS
#define MK_NT_LOADS 1
#endif
#ifndef MK_DOT2_BUILTIN
#define MK_DOT2_BUILTIN 0
#endif

namespace {

constexpr int kThreads = MK_THREADS;
constexpr int kWaves = kThreads / 64;
constexpr int kChunkElems = 512;  // bf16 columns covered by one wave-wide 16 B/lane load
// More than half of the 160 KiB LDS: the dispatcher can then place only one
// workgroup per compute unit, so a grid of #CU workers covers every CU once.
constexpr int kMinLdsBytes = 84 * 1024;
constexpr uint32_t kTicksPerUs = 100;  // s_memrealtime runs at 100 MHz

static_assert(kThreads % 64 == 0 && kThreads <= 1024, "wave64 workgroup");

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));

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
};

// Per-workgroup state that outlives a single instruction.
struct SharedState {
    float red[kWaves * MK_MAX_EXPERTS];
    float logits[MK_MAX_EXPERTS];
    int route_layer;  // layer whose routing below was computed here, -1 none
    int route_idx[2];
    float route_score[2];  // bf16 score values widened to fp32
    int flag;
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
#if MK_DOT2_BUILTIN
    acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, w.x), __builtin_bit_cast(bf16x2, a.x), acc, false);
    acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, w.y), __builtin_bit_cast(bf16x2, a.y), acc, false);
    acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, w.z), __builtin_bit_cast(bf16x2, a.z), acc, false);
    acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, w.w), __builtin_bit_cast(bf16x2, a.w), acc, false);
#else
    acc = dot2_fma(w.x, a.x, acc);
    acc = dot2_fma(w.y, a.y, acc);
    acc = dot2_fma(w.z, a.z, acc);
    acc = dot2_fma(w.w, a.w, acc);
#endif
    return acc;
}

// Butterfly sum over the 64 lanes; every lane ends with the same value
// (each step adds the same two operands on both partner lanes).
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) v += __shfl_xor(v, m, 64);
    return v;
}

__device__ __forceinline__ float block_sum(float v, float *red) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    v = wave_sum(v);
    if (lane == 0) red[wave] = v;
    __syncthreads();
    float s = 0.f;
#pragma unroll
    for (int i = 0; i < kWaves; ++i) s += red[i];
    __syncthreads();
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

__device__ __forceinline__ int32_t *bar_at(const KParams &p, int layer, int opcode) {
    return p.bar + ((size_t)layer * p.bar_ops + (opcode - 1)) * p.bar_width;
}

__device__ __forceinline__ bool aborted(const KParams &p) {
    return __hip_atomic_load(p.status, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != 0;
}

// Record the first failure (thread 0 of the reporting workgroup only).
__device__ void report_error(const KParams &p, int code, const Ctx &c, int opcode, int layer, int expected, int seen) {
    if (threadIdx.x != 0) return;
    int zero = 0;
    if (__hip_atomic_compare_exchange_strong(p.status, &zero, code, __ATOMIC_RELAXED, __ATOMIC_RELAXED,
                                             __HIP_MEMORY_SCOPE_AGENT)) {
        p.status[MK_STATUS_WORKER] = c.worker;
        p.status[MK_STATUS_SLOT] = c.slot;
        p.status[MK_STATUS_OPCODE] = opcode;
        p.status[MK_STATUS_LAYER] = layer;
        p.status[MK_STATUS_EXPECTED] = expected;
        p.status[MK_STATUS_SEEN] = seen;
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
    }
}

// Wait until *ctr >= expected.  Thread 0 spins; the result is broadcast.
// Returns false (uniformly) on time-out or when another worker has failed.
__device__ bool wait_ge(const KParams &p, SharedState &sh, int32_t *ctr, int expected, const Ctx &c, int opcode,
                        int layer) {
    if (threadIdx.x == 0) {
        int ok = 1;
        int v = __hip_atomic_load(ctr, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (v < expected) {
            const uint64_t t0 = __builtin_amdgcn_s_memrealtime();
            for (;;) {
                __builtin_amdgcn_s_sleep(1);
                v = __hip_atomic_load(ctr, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
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
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
        sh.flag = ok;
    }
    __syncthreads();
    const bool ok = sh.flag != 0;
    __syncthreads();
    return ok;
}

// Make every wave's global stores complete, then join the workgroup.  A
// workgroup barrier alone does not wait for outstanding stores of other
// waves, and the release below only writes back what has reached L2.
__device__ __forceinline__ void drain_and_sync() {
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
}

__device__ __forceinline__ void arrive(int32_t *ctr, int n) {
    if (threadIdx.x == 0) __hip_atomic_fetch_add(ctr, n, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_AGENT);
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

// ---------------------------------------------------------------------------
// RMSNorm + router (shared by opcodes 5 and 8)
// ---------------------------------------------------------------------------

// normed hidden (bf16) -> act[0 .. H/8); router logits -> sh.logits[0 .. E).
__device__ void rms_router(const KParams &p, SharedState &sh, u32x4 *act, int layer, const uint16_t *router) {
    const int tid = threadIdx.x;
    const int nv = p.H >> 3;
    const u32x4 *x4 = reinterpret_cast<const u32x4 *>(p.hidden);
    const u32x4 *w4 = reinterpret_cast<const u32x4 *>(p.ffn_ln + (size_t)layer * p.H);

    float ss = 0.f;
    for (int v = tid; v < nv; v += kThreads) {
        const u32x4 x = x4[v];
        ss += sumsq2(x.x) + sumsq2(x.y) + sumsq2(x.z) + sumsq2(x.w);
    }
    ss = block_sum(ss, sh.red);
    const float r = 1.0f / sqrtf(ss / (float)p.H + p.eps);

    const uint16_t *rw = router + (size_t)layer * p.E * p.H;
    float acc[MK_MAX_EXPERTS];
#pragma unroll
    for (int e = 0; e < MK_MAX_EXPERTS; ++e) acc[e] = 0.f;
    for (int v = tid; v < nv; v += kThreads) {
        const u32x4 x = x4[v], w = w4[v];
        u32x4 n;
        n.x = norm2(x.x, w.x, r);
        n.y = norm2(x.y, w.y, r);
        n.z = norm2(x.z, w.z, r);
        n.w = norm2(x.w, w.w, r);
        act[v] = n;
#pragma unroll
        for (int e = 0; e < MK_MAX_EXPERTS; ++e)
            if (e < p.E) acc[e] = dot8(reinterpret_cast<const u32x4 *>(rw + (size_t)e * p.H)[v], n, acc[e]);
    }
    const int lane = tid & 63, wave = tid >> 6;
#pragma unroll
    for (int e = 0; e < MK_MAX_EXPERTS; ++e) {
        if (e < p.E) {
            const float s = wave_sum(acc[e]);
            if (lane == 0) sh.red[e * kWaves + wave] = s;
        }
    }
    __syncthreads();
    if (tid < p.E) {
        float s = 0.f;
#pragma unroll
        for (int i = 0; i < kWaves; ++i) s += sh.red[tid * kWaves + i];
        if (p.router_bias != nullptr) s += p.router_bias[layer * p.E + tid];
        sh.logits[tid] = s;
    }
    __syncthreads();
}

struct Top2 {
    int i0, i1;
    float p0, p1;
};

// softmax over E logits, then the two largest probabilities in descending
// order (strict comparison: the lower expert index wins a tie).
__device__ Top2 softmax_top2(const float *logits, int E) {
    float m = logits[0];
    for (int e = 1; e < E; ++e) m = fmaxf(m, logits[e]);
    float s = 0.f;
    for (int e = 0; e < E; ++e) s += expf(logits[e] - m);
    Top2 t{0, -1, expf(logits[0] - m) / s, -1.f};
    for (int e = 1; e < E; ++e) {
        const float pe = expf(logits[e] - m) / s;
        if (pe > t.p0) {
            t.i1 = t.i0;
            t.p1 = t.p0;
            t.i0 = e;
            t.p0 = pe;
        } else if (t.i1 < 0 || pe > t.p1) {
            t.i1 = e;
            t.p1 = pe;
        }
    }
    return t;
}

// ---------------------------------------------------------------------------
// opcode 5: RmsRouterUpgate  (python_vm.py:228-277)
// ---------------------------------------------------------------------------

__device__ bool op_rms_router_upgate(const KParams &p, SharedState &sh, u32x4 *act, const int32_t *ins,
                                     const Ctx &c, int32_t *tim) {
    const int layer = __builtin_amdgcn_readfirstlane(ins[1]);
    const int start = __builtin_amdgcn_readfirstlane(ins[2]);
    const int nb = __builtin_amdgcn_readfirstlane(ins[3]);
    if (layer < 0 || layer >= p.num_layers || start < 0 || nb < 0 ||
        (int64_t)(start + nb) * p.expert_bs > (int64_t)p.F) {
        report_error(p, MK_ERR_BAD_INSTRUCTION, c, 5, layer, start, nb);
        return false;
    }
    stamp(tim, MK_TEVENT_AT_GMEM_WAIT);
    if (!wait_ge(p, sh, bar_at(p, layer, 4), p.H / p.oproj_bs, c, 5, layer)) return false;
    stamp(tim, MK_TEVENT_DONE_GMEM_WAIT);

    rms_router(p, sh, act, layer, p.router);
    const Top2 t = softmax_top2(sh.logits, p.E);
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
    if (start == 0) {
        u32x4 *out = reinterpret_cast<u32x4 *>(p.normed_out);
        for (int v = tid; v < (p.H >> 3); v += kThreads) out[v] = act[v];
        if (tid == 0) {
            p.sel_idx[0] = t.i0;
            p.sel_idx[1] = t.i1;
            p.sel_score[0] = (uint16_t)sc0;
            p.sel_score[1] = (uint16_t)sc1;
        }
    }
    stamp(tim, MK_TEVENT_FIRST_LOAD);

    const int lane = tid & 63, wave = tid >> 6;
    const int row0 = start * p.expert_bs, nrows = nb * p.expert_bs;
    const int nc = p.H / kChunkElems;
    for (int it = wave; it < 2 * nrows; it += kWaves) {
        const int j = it >= nrows;
        const int r = row0 + (j ? it - nrows : it);
        const int e = j ? t.i1 : t.i0;
        const size_t off = ((size_t)(layer * p.E + e) * p.F + r) * (size_t)p.H;
        float ag = 0.f, au = 0.f;
        dot_pair(p.gate + off, p.up + off, act, act, nc, lane, ag, au);
        ag = wave_sum(ag);
        au = wave_sum(au);
        if (lane == 0) {
            const float g = rbf(ag), u = rbf(au);
            const float sg = rbf(g / (1.0f + expf(-g)));
            p.silu[(size_t)e * p.F + r] = (uint16_t)f2bf(sg * u);
        }
    }
    drain_and_sync();
    arrive(bar_at(p, layer, 5), nb);
    stamp(tim, MK_TEVENT_DONE_GMEM_STORE);
    return true;
}

// ---------------------------------------------------------------------------
// opcode 6: ExpertDownProjFused  (python_vm.py:284-314)
// ---------------------------------------------------------------------------

__device__ bool op_expert_downproj(const KParams &p, SharedState &sh, u32x4 *act, const int32_t *ins,
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
    stamp(tim, MK_TEVENT_AT_GMEM_WAIT);
    if (!wait_ge(p, sh, bar_at(p, layer, 5), p.F / p.expert_bs, c, 6, layer)) return false;
    stamp(tim, MK_TEVENT_DONE_GMEM_WAIT);

    int e0, e1;
    float s0, s1;
    if (sh.route_layer == layer) {
        e0 = sh.route_idx[0];
        e1 = sh.route_idx[1];
        s0 = sh.route_score[0];
        s1 = sh.route_score[1];
    } else {
        e0 = __builtin_amdgcn_readfirstlane(p.sel_idx[0]);
        e1 = __builtin_amdgcn_readfirstlane(p.sel_idx[1]);
        s0 = bf2f(p.sel_score[0]);
        s1 = bf2f(p.sel_score[1]);
    }
    if (e0 < 0 || e0 >= p.E || e1 < 0 || e1 >= p.E) {
        report_error(p, MK_ERR_BAD_INSTRUCTION, c, 6, layer, e0, e1);
        return false;
    }

    const int tid = threadIdx.x;
    const int nv = p.F >> 3;
    const u32x4 *a0 = reinterpret_cast<const u32x4 *>(p.silu + (size_t)e0 * p.F);
    const u32x4 *a1 = reinterpret_cast<const u32x4 *>(p.silu + (size_t)e1 * p.F);
    for (int v = tid; v < nv; v += kThreads) {
        act[v] = a0[v];
        act[nv + v] = a1[v];
    }
    __syncthreads();
    stamp(tim, MK_TEVENT_FIRST_LOAD);

    const int lane = tid & 63, wave = tid >> 6;
    const int row0 = start * p.down_bs, nrows = (end - start) * p.down_bs;
    const int nc = p.F / kChunkElems;
    const size_t base0 = (size_t)(layer * p.E + e0) * p.H;
    const size_t base1 = (size_t)(layer * p.E + e1) * p.H;
    for (int it = wave; it < nrows; it += kWaves) {
        const int r = row0 + it;
        float d0 = 0.f, d1 = 0.f;
        dot_pair(p.down + (base0 + r) * (size_t)p.F, p.down + (base1 + r) * (size_t)p.F, act, act + nv, nc, lane,
                 d0, d1);
        d0 = wave_sum(d0);
        d1 = wave_sum(d1);
        if (lane == 0) {
            float h = bf2f(p.hidden[r]);
            h = rbf(h + rbf(s0 * rbf(d0)));
            h = rbf(h + rbf(s1 * rbf(d1)));
            p.hidden[r] = (uint16_t)f2bf(h);
        }
    }
    drain_and_sync();
    arrive(bar_at(p, layer, 6), 2 * (end - start));
    stamp(tim, MK_TEVENT_DONE_GMEM_STORE);
    return true;
}

// ---------------------------------------------------------------------------
// opcode 8: SpeculativeExpertPredict  (python_vm.py:356-371)
// ---------------------------------------------------------------------------

__device__ bool op_predict(const KParams &p, SharedState &sh, u32x4 *act, const int32_t *ins, const Ctx &c,
                           int32_t *tim) {
    const int layer = __builtin_amdgcn_readfirstlane(ins[1]);
    if (layer < 0 || layer >= p.num_layers) {
        report_error(p, MK_ERR_BAD_INSTRUCTION, c, 8, layer, 0, 0);
        return false;
    }
    if (layer > 0) {
        stamp(tim, MK_TEVENT_AT_GMEM_WAIT);
        if (!wait_ge(p, sh, bar_at(p, layer - 1, 6), 2 * (p.H / p.down_bs), c, 8, layer)) return false;
        stamp(tim, MK_TEVENT_DONE_GMEM_WAIT);
    }
    rms_router(p, sh, act, layer, p.predictor != nullptr ? p.predictor : p.router);
    const Top2 t = softmax_top2(sh.logits, p.E);
    if (threadIdx.x == 0) {
        p.pred_idx[0] = t.i0;
        p.pred_idx[1] = t.i1;
    }
    drain_and_sync();
    arrive(bar_at(p, layer, 8), 1);
    stamp(tim, MK_TEVENT_DONE_GMEM_STORE);
    return true;
}

// ---------------------------------------------------------------------------
// the persistent interpreter
// ---------------------------------------------------------------------------

__global__ void __launch_bounds__(kThreads) mk_mixtral_kernel(KParams p) {
    extern __shared__ u32x4 act[];
    __shared__ SharedState sh;
    if (threadIdx.x == 0) sh.route_layer = -1;
    __syncthreads();

    const int w = blockIdx.x;
    for (int q = 0; q < p.queue_len; ++q) {
        const size_t slot = (size_t)w * p.queue_len + q;
        const int32_t *ins = p.instructions + slot * MK_INTS_PER_INSTRUCTION;
        int32_t *tim = p.timings != nullptr ? p.timings + slot * MK_TIMING_SLOTS : nullptr;
        const int op = __builtin_amdgcn_readfirstlane(ins[0]);
        const Ctx c{w, q};
        stamp(tim, MK_TEVENT_START);
        bool ok = true;
        switch (op) {
        case 0: break;
        case 5: ok = op_rms_router_upgate(p, sh, act, ins, c, tim); break;
        case 6: ok = op_expert_downproj(p, sh, act, ins, c, tim); break;
        case 8: ok = op_predict(p, sh, act, ins, c, tim); break;
        case 1:
        case 2:
        case 3:
        case 4:
        case 7:
            report_error(p, MK_ERR_UNSUPPORTED_OPCODE, c, op, __builtin_amdgcn_readfirstlane(ins[1]), 0, op);
            ok = false;
            break;
        default:
            report_error(p, MK_ERR_BAD_OPCODE, c, op, 0, 0, op);
            ok = false;
            break;
        }
        stamp(tim, MK_TEVENT_END);
        if (!ok) break;
    }
}

// ---------------------------------------------------------------------------
// host side
// ---------------------------------------------------------------------------

constexpr int kMaxDevices = 64;

struct DeviceState {
    bool ready = false;
    int num_cus = 0;
    int max_lds = 0;
    int32_t *status = nullptr;
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

// `dev` must be the current device.
int device_state(int dev, DeviceState **out) {
    if (dev < 0 || dev >= kMaxDevices) return MK_ERR_INVALID_ARGUMENT;
    std::lock_guard<std::mutex> lock(g_mutex);
    DeviceState &st = g_devices[dev];
    if (!st.ready) {
        hipError_t e = hipDeviceGetAttribute(&st.num_cus, hipDeviceAttributeMultiprocessorCount, dev);
        if (e != hipSuccess) return hip_fail(e, "hipDeviceGetAttribute");
        e = hipDeviceGetAttribute(&st.max_lds, hipDeviceAttributeMaxSharedMemoryPerBlock, dev);
        if (e != hipSuccess) return hip_fail(e, "hipDeviceGetAttribute");
        e = hipMalloc(reinterpret_cast<void **>(&st.status), MK_STATUS_WORDS * sizeof(int32_t));
        if (e != hipSuccess) return hip_fail(e, "hipMalloc");
        e = hipMemset(st.status, 0, MK_STATUS_WORDS * sizeof(int32_t));
        if (e != hipSuccess) return hip_fail(e, "hipMemset");
        st.ready = true;
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

size_t lds_bytes_for(const mk_mixtral_globals *g) {
    const size_t normed = (size_t)g->hidden_size * 2;
    const size_t silu = (size_t)g->intermediate_size * 2 * 2;
    size_t need = normed > silu ? normed : silu;
    return need > (size_t)kMinLdsBytes ? need : (size_t)kMinLdsBytes;
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
        g->intermediate_size % kChunkElems)
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
    return MK_OK;
}

}  // namespace

extern "C" {

int mk_mixtral_abi_version(void) { return MK_MIXTRAL_ABI_VERSION; }

int mk_mixtral_last_hip_error(void) { return g_last_hip_error; }

const char *mk_mixtral_last_error_site(void) { return g_last_hip_site; }

const char *mk_mixtral_error_string(int code) {
    switch (code) {
    case MK_OK: return "ok";
    case MK_ERR_INVALID_ARGUMENT: return "invalid argument";
    case MK_ERR_UNSUPPORTED: return "shape or configuration not supported by the kernel";
    case MK_ERR_HIP: return "HIP runtime error";
    case MK_ERR_NOT_CORESIDENT: return "worker count exceeds co-resident workgroups";
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
        &blocks, reinterpret_cast<const void *>(mk_mixtral_kernel), kThreads, kMinLdsBytes);
    if (e != hipSuccess) return hip_fail(e, "hipOccupancyMaxActiveBlocksPerMultiprocessor");
    if (num_cus) *num_cus = st->num_cus;
    if (max_workers) *max_workers = blocks * st->num_cus;
    return MK_OK;
}

int mk_mixtral_launch(const mk_mixtral_globals *g, void *stream) {
    int rc = validate(g);
    if (rc != MK_OK) return rc;
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return hip_fail(e, "hipGetDevice");
    DeviceState *st = nullptr;
    rc = device_state(dev, &st);
    if (rc != MK_OK) return rc;

    const size_t lds = lds_bytes_for(g);
    if (lds + sizeof(SharedState) > (size_t)st->max_lds) return MK_ERR_UNSUPPORTED;
    int blocks = 0;
    e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&blocks, reinterpret_cast<const void *>(mk_mixtral_kernel),
                                                     kThreads, lds);
    if (e != hipSuccess) return hip_fail(e, "hipOccupancyMaxActiveBlocksPerMultiprocessor");
    if (g->num_workers > (int64_t)blocks * st->num_cus) return MK_ERR_NOT_CORESIDENT;

    KParams kp;
    kp.instructions = g->instructions;
    kp.timings = g->record_timings ? g->timings : nullptr;
    kp.bar = g->barriers;
    kp.status = g->status != nullptr ? g->status : st->status;
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
    kp.expert_bs = g->expert_proj_block_size;
    kp.down_bs = g->down_proj_block_size;
    kp.oproj_bs = g->o_proj_block_size;
    kp.eps = g->rms_norm_eps;
    const uint64_t us = g->spin_timeout_us ? g->spin_timeout_us : 2000000u;
    const uint64_t ticks = us * kTicksPerUs;
    kp.timeout_ticks = ticks > 0xffffffffu ? 0xffffffffu : (uint32_t)ticks;

    hipLaunchKernelGGL(mk_mixtral_kernel, dim3((unsigned)g->num_workers), dim3(kThreads), lds,
                       reinterpret_cast<hipStream_t>(stream), kp);
    e = hipGetLastError();
    if (e != hipSuccess) return hip_fail(e, "hipGetLastError");
    return MK_OK;
}

int mk_mixtral_read_status(int device, int32_t *out) {
    if (out == nullptr) return MK_ERR_INVALID_ARGUMENT;
    DeviceGuard guard(device);
    if (guard.err != hipSuccess) return hip_fail(guard.err, "hipSetDevice");
    DeviceState *st = nullptr;
    int rc = device_state(device, &st);
    if (rc != MK_OK) return rc;
    hipError_t e = hipDeviceSynchronize();
    if (e == hipSuccess) e = hipMemcpy(out, st->status, MK_STATUS_WORDS * sizeof(int32_t), hipMemcpyDeviceToHost);
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
    if (e == hipSuccess) e = hipDeviceSynchronize();
    if (e != hipSuccess) return hip_fail(e, "hipDeviceSynchronize");
    return MK_OK;
}

}  // extern "C"
