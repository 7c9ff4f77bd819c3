/*
 * mk_mixtral.h -- C ABI of the MI355X (gfx950) persistent MoE decode
 * megakernel.
 *
 * Replaces the reference's pybind11 binding `mk_mixtral(...)`
 * (demos/mixtral/mixtral.cu:28-94), whose argument order is the field order
 * of `mixtral_globals` (demos/mixtral/mixtral.cuh:153-203) and of the Python
 * caller `interpret_with_mk` (megakernels/mixtral/mk.py:42-96).  The struct
 * below keeps that field order; tensors become raw device pointers plus the
 * dimensions the reference bakes in at compile time
 * (demos/mixtral/mixtral.cuh:22-35).
 *
 * Conventions
 *   - bf16 tensors are passed as `uint16_t *` (raw bf16 bit patterns).
 *   - Every pointer is a device pointer on the current HIP device, except
 *     where noted.  The caller owns all memory; the kernel only borrows it.
 *   - Launches are asynchronous on `stream` (a `hipStream_t`, NULL = default
 *     stream).  Entry points never throw; they return an `mk_status_code`.
 *   - Launches on one device run one at a time, in the order they are made
 *     (from any host thread, mk_llama_launch included): a persistent kernel
 *     needs every workgroup resident at once, and the library's scratch and
 *     status words are per device.  A launch on a stream other than the
 *     previous launch's makes its stream wait (hipStreamWaitEvent) for all
 *     work queued on that previous stream so far; if that stream has been
 *     destroyed, the launch synchronises the device first.  Work on the
 *     previous stream queued after the wait is not waited for.
 *   - The caller zeroes (or pre-fills) `barriers` before each launch, as the
 *     reference's callers do (megakernels/generators.py:115-116,132).
 *
 * Instruction queues: `instructions[num_workers][queue_len][32]` int32, the
 * serialised layout of megakernels/instructions.py:97-119.  Worker w (one
 * workgroup, one compute unit) runs queue w in order.  Opcodes:
 *   0 NoOp
 *   1 Mixtral_QKV               [1, layer, start_block, end_block]
 *   2 Mixtral_PartialAttn       [2, layer, kv_head, num_partials, partial_idx]
 *   3 Mixtral_AttnReduction     [3, layer, head_start, num_partials, is_terminal,
 *                                n, list[n]..., output_partial_idx]
 *   4 Mixtral_OProj             [4, layer, start_block, end_block, reduction_block=0]
 *   5 RmsRouterUpgate           [5, layer, start_block, num_blocks]
 *   6 ExpertDownProjFused       [6, layer, start_block, end_block, reduction_block=0]
 *   7 Mixtral_RMS_LM_Head       [7, start_block, end_block, reduction_block]
 *   8 SpeculativeExpertPredict  [8, layer]
 * Opcodes 1-4 and 7 need the attention tensors (qkv_weights non-NULL);
 * without them they are rejected with MK_ERR_UNSUPPORTED_OPCODE.
 *
 * Barriers: `barriers[bar_layers][bar_ops][bar_width]` int32, counter for
 * (layer, opcode) at [layer][opcode-1][idx].  Waits proceed once a counter is
 * >= the expected arrival count (so pre-filled barriers satisfy them):
 *   opcode 1 waits [l-1][5][0] >= k * hidden / down_proj_block_size (l > 0)
 *   opcode 2 waits [l][0][h] >= head_dim / qkv_block_size for its heads
 *   opcode 3 waits [l][1][head_start] >= num_partials
 *   opcode 4 waits [l][2][0] >= num_attention_heads
 *   opcode 5 waits [l][3][0] >= hidden / o_proj_block_size
 *   opcode 6 waits [l][4][0] >= intermediate / expert_proj_block_size
 *   opcode 7 waits [L-1][5][0] >= k * hidden / down_proj_block_size
 *   opcode 8 waits [l-1][5][0] >= k * hidden / down_proj_block_size (l > 0)
 * and arrive as megakernels/mixtral/python_vm.py:38-371 does.
 *
 * Device-side failures (barrier spin time-out, bad opcode or operand) are
 * recorded in a status word and make every worker exit; they are read back
 * with mk_mixtral_read_status().
 */
#ifndef MK_MIXTRAL_H
#define MK_MIXTRAL_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define MK_MIXTRAL_ABI_VERSION 5
#define MK_INTS_PER_INSTRUCTION 32
#define MK_TIMING_SLOTS 128
#define MK_STATUS_WORDS 16
#define MK_MAX_EXPERTS 16

typedef enum mk_status_code {
    MK_OK = 0,
    MK_ERR_INVALID_ARGUMENT = 1,  /* host validation failed                   */
    MK_ERR_UNSUPPORTED = 2,       /* shape outside what the kernel implements */
    MK_ERR_HIP = 3,               /* HIP runtime error, see mk_mixtral_last_hip_error */
    MK_ERR_NOT_CORESIDENT = 4,    /* grid cannot be fully resident            */
    MK_ERR_SCRATCH_TOO_SMALL = 5, /* mk_mixtral_launch_noalloc: the launch needs
                                     more than its fixed scratch holds       */
    MK_ERR_TIMEOUT = 16,          /* device: barrier spin timed out           */
    MK_ERR_BAD_OPCODE = 17,       /* device: opcode not in 0..8               */
    MK_ERR_UNSUPPORTED_OPCODE = 18, /* device: opcode 1-4 or 7                */
    MK_ERR_BAD_INSTRUCTION = 19   /* device: operand out of range             */
} mk_status_code;

/* Status words written by the kernel (first failure wins):
 * [0] code, [1] worker, [2] queue slot, [3] opcode, [4] layer,
 * [5] expected count / bad word index, [6] observed count / bad value. */
enum {
    MK_STATUS_CODE = 0,
    MK_STATUS_WORKER = 1,
    MK_STATUS_SLOT = 2,
    MK_STATUS_OPCODE = 3,
    MK_STATUS_LAYER = 4,
    MK_STATUS_EXPECTED = 5,
    MK_STATUS_SEEN = 6
};

/* Timing slots (subset of include/util.cuh:220-252 of the reference), in
 * 100 MHz s_memrealtime ticks (low 32 bits, global clock shared by all
 * compute units) when timing is enabled. */
enum {
    MK_TEVENT_START = 0,
    MK_TEVENT_END = 4,
    MK_TEVENT_AT_GMEM_WAIT = 44,
    MK_TEVENT_DONE_GMEM_WAIT = 45,
    MK_TEVENT_AT_GMEM_STORE = 46,
    MK_TEVENT_DONE_GMEM_STORE = 47,
    MK_TEVENT_FIRST_LOAD = 48,
    MK_TEVENT_FIRST_USE = 49,
    /* opcode 5 of a whole-model launch: the experts opcode 8 predicted and
     * the ones selected, one byte each (predicted 0, 1, selected 0, 1 from
     * the low byte up; 0xff = no prediction) -- not a time */
    MK_TEVENT_PREDICTION = 50
    /* also written, as times: 52-53 inside opcode 3 (weights in LDS, sums
     * stored), 55-56 inside opcode 2 (wave partials in LDS, merged outputs
     * stored), 60-63 inside the RMSNorm + router of opcodes 5 and 8, 64-95
     * per-item completions of opcode 5 (waves 0 and 7, 16 items each) */
};

typedef struct mk_mixtral_globals {
    uint32_t struct_size;          /* sizeof(mk_mixtral_globals) */
    uint32_t abi_version;          /* MK_MIXTRAL_ABI_VERSION */

    /* megakernel internals (mixtral.cuh:155-157) */
    int32_t *barriers;             /* [bar_layers, bar_ops, bar_width] */
    int64_t bar_layers, bar_ops, bar_width;
    const int32_t *instructions;   /* [num_workers, queue_len, 32] */
    int64_t num_workers, queue_len;
    int32_t *timings;              /* [num_workers, queue_len, 128] or NULL */

    /* attention weights (mixtral.cuh:160-162), bf16, NULL if absent */
    const uint16_t *qkv_weights;        /* [L, (Hq + 2 Hkv) D, H] */
    const uint16_t *attn_norm_weights;  /* [L, H]                 */
    const uint16_t *o_weights;          /* [L, H, Hq D]           */

    /* MoE weights (mixtral.cuh:165-169), bf16, row-major */
    const uint16_t *expert_gate_weights;  /* [L*E, F, H] */
    const uint16_t *expert_up_weights;    /* [L*E, F, H] */
    const uint16_t *expert_down_weights;  /* [L*E, H, F] */
    const uint16_t *router_weights;       /* [L*E, H]    */
    const uint16_t *ffn_ln_weights;       /* [L, H]      */

    /* LM head, KV cache, RoPE (mixtral.cuh:172-181) */
    const uint16_t *lm_head_norm_weights;  /* [H] bf16                     */
    const uint16_t *lm_head_weights;       /* [V, H] bf16                  */
    uint16_t *k_cache;                     /* [L, T, Hkv, D] bf16          */
    uint16_t *v_cache;                     /* [L, T, Hkv, D] bf16          */
    const float *rope_cos;                 /* [T, D] fp32, interleaved     */
    const float *rope_sin;                 /* [T, D] fp32                  */

    /* activations (mixtral.cuh:184-191) */
    uint16_t *hidden_states;       /* [H] bf16, updated in place by opcodes 4 and 6 */
    uint16_t *q_post_rope;         /* [Hq D] bf16                 */
    uint16_t *attn_out;            /* [Hq D] bf16                 */
    float *attn_lse_intermediates; /* [Hq, P] fp32                */
    float *attn_out_intermediates; /* [Hq, P, D] fp32             */
    uint16_t *expert_silu_out;     /* [E, F] bf16 */
    uint16_t *router_normed_hidden;/* [H] bf16 */
    uint16_t *logits;              /* [V] bf16, accumulated by opcode 7 (caller zeroes) */

    /* router outputs (mixtral.cuh:194-198) */
    int32_t *selected_expert_indices;   /* [k] */
    uint16_t *selected_expert_scores;   /* [k] bf16 */
    int32_t *predicted_expert_indices;  /* [k] */

    /* scalars (mixtral.cuh:201-204) */
    uint32_t pos_id;
    float attn_scale;
    float rms_norm_eps;
    int32_t skip_attn_reduction;

    /* dimensions compiled into the reference kernel (mixtral.cuh:22-35) */
    int32_t num_layers;
    int32_t hidden_size;           /* H, multiple of 512 */
    int32_t intermediate_size;     /* F, multiple of 512 */
    int32_t num_experts;           /* E, 2..16 */
    int32_t num_experts_per_tok;   /* k, must be 2 */

    /* block sizes (MixtralGlobals fields, megakernels/mixtral/scheduler.py:144-151) */
    int32_t expert_proj_block_size;
    int32_t down_proj_block_size;
    int32_t o_proj_block_size;

    /* attention and LM-head shape (compiled into the reference kernel,
     * demos/mixtral/mixtral.cuh:22-35; MixtralGlobals block sizes).  Only read
     * by opcodes 1-4 and 7; all zero when the attention tensors are absent. */
    int32_t qkv_block_size;        /* rows per QKV block (16)                */
    int32_t attn_kv_block_size;    /* KV positions per attention block (16)  */
    int32_t lm_head_block_size;    /* logit rows per LM-head block (16)      */
    int32_t lm_head_reduction;     /* columns per LM-head reduction block (2048) */
    int32_t num_attention_heads;   /* Hq                                     */
    int32_t num_kv_heads;          /* Hkv; Hq / Hkv in 1..4                  */
    int32_t head_dim;              /* D: 64 or 128                           */
    int32_t vocab_size;            /* V                                      */
    int32_t kv_capacity;           /* T: positions per layer in the KV cache */
    int32_t attn_partial_slots;    /* P: columns of attn_*_intermediates     */

    /* extensions, no counterpart in the reference; NULL keeps its semantics */
    const float *router_bias;          /* [L*E] fp32 added to router logits  */
    const uint16_t *predictor_weights; /* [L*E, H] bf16 for opcode 8        */

    /* control */
    int32_t *status;               /* device int32[16], NULL = library-owned buffer */
    uint32_t spin_timeout_us;      /* barrier spin limit, 0 = 2 s            */
    int32_t record_timings;        /* nonzero: write timing slots           */
    int32_t work_sharing;          /* zero: each instruction does exactly its
                                      own rows; nonzero: idle workers also take
                                      unclaimed rows of other opcode-5
                                      instructions of the same layer (same
                                      results, same barrier counts) */

    /* decode-driver extension, no counterpart in the reference kernel: its
     * generator takes torch.argmax of the logits and embeds the token between
     * launches (megakernels/generators.py:121-145).  NULL keeps the reference
     * semantics; both need the LM head (attention tensors present). */
    int64_t *argmax_out;           /* when the launch ends: argmax of logits, the
                                      first maximal index (NaN counts as
                                      maximal, as in torch.argmax) */
    const uint16_t *next_embed_weights; /* [V, H] bf16, needs argmax_out: when
                                      the launch ends, hidden_states := row
                                      *argmax_out (the next step's input) */
    int32_t reset_for_next_launch; /* nonzero: when the launch ends, the
                                      barrier tensor (its num_layers layers)
                                      and the logits are zeroed, so the next
                                      launch needs no fill; the caller then
                                      cannot read either */

    /* opcode-5/6 overlap, no counterpart in the reference (its opcode 6
     * waits for every opcode-5 block).  Nonzero, and work_sharing zero:
     * opcode 5 also counts finished SiLU rows per 512-row chunk of F in the
     * library's scratch, and opcode 6 starts on groups of 4 chunks as they
     * complete, on a workgroup that routed the layer itself.  Same indices,
     * scores and barrier counts; hidden_states differ from the zero setting
     * only in the fp32 summation order of each row.  Pairs with an opcode-5
     * partition whose blocks interleave across workers (worker w: blocks
     * w, w + W, ...), which makes column chunks complete early.  Applies to
     * MoE-only launches (qkv_weights NULL) with 8 experts; ignored
     * otherwise. */
    int32_t downproj_overlap;

    /* prefetch switch, no reference counterpart as a field (the reference
     * always prefetches the predicted experts, demos/mixtral/
     * rms_router_matvec.cu:259-290).  Nonzero: every instruction waits for
     * its inputs before it issues any load (weights, KV rows, router rows),
     * no predicted expert rows are staged, and opcode 6 takes no early
     * loads; same results.  For prefetch on/off comparisons of whole-model
     * launches (qkv_weights non-NULL); MoE-only launches ignore it. */
    int32_t late_loads;
} mk_mixtral_globals;

/* Launch one persistent-kernel pass over the instruction queues.
 * Replaces the pybind11 `mk_mixtral` (demos/mixtral/mixtral.cu:28-94). */
int mk_mixtral_launch(const mk_mixtral_globals *g, void *stream);

/* Launch like mk_mixtral_launch, allocating nothing: no hipMalloc, hipFree,
 * event or other allocating call, on any call (the first on a device
 * included).  No counterpart in the reference: for callers that cannot
 * allocate -- code under HIP graph capture, tight serving loops, harnesses
 * that forbid allocation.  The caller still passes every input and output.
 *   - The launch's scratch (exit counter, two ints of work-sharing cursors
 *     per instruction slot, column-chunk counters, spread layer counters)
 *     lives in a fixed 2 MiB device array per device, held until the process
 *     ends.  A launch that needs more -- about 2 x num_workers x queue_len
 *     + 8 x 1024 ints -- returns MK_ERR_SCRATCH_TOO_SMALL without launching
 *     (up to about 250000 instruction slots, e.g. 256 workers x 980).
 *   - With `status` NULL, the status words are 16 ints of that array;
 *     mk_mixtral_read_status / mk_mixtral_clear_status cover them.
 *   - Every call on a device shares the array, and each launch leaves it
 *     zeroed when its last workgroup exits.  Calls that overlap on one GPU
 *     race: unlike mk_mixtral_launch, this entry point records and waits on
 *     no event, so the caller orders it after launches on other streams
 *     (one stream for all launches does that).  Nor does a later
 *     mk_mixtral_launch order itself after a no-allocation launch (its
 *     stream may be capturing a graph): it follows the previous
 *     mk_mixtral_launch only, and the caller orders the two kinds. */
int mk_mixtral_launch_noalloc(const mk_mixtral_globals *g, void *stream);

/* Copy the library-owned status words of `device` into out[16] after a
 * device-wide synchronisation.  No reference counterpart (the reference has
 * no device-side error reporting). */
int mk_mixtral_read_status(int device, int32_t *out);

/* Zero the library-owned status words of `device` (synchronous). */
int mk_mixtral_clear_status(int device);

/* Number of compute units and the largest worker count that can be
 * co-resident for this kernel.  Counterpart of get_sm_count
 * (megakernels/utils.py:133-135). */
int mk_mixtral_query_device(int device, int32_t *num_cus, int32_t *max_workers);

/* Read the launch-time tuning overrides (MK_SPREAD, MK_SPIN_SLEEP, MK_TAIL,
 * MK_EARLY, MK_PF, MK_STAGE_ITEMS) from the environment again.  No
 * reference counterpart: these are measurement settings of this build.  The
 * library reads them once per process, at its first launch; a value that is
 * not a whole number is ignored with a warning, and each override in effect
 * is reported on stderr when read.  Shared by mk_mixtral_launch,
 * mk_mixtral_launch_noalloc and mk_llama_launch; call it while no launch is
 * being made from another thread. */
void mk_mixtral_reload_overrides(void);

const char *mk_mixtral_error_string(int code);
/* hipError_t and the name of the HIP call behind the last MK_ERR_HIP on the
 * calling thread. */
int mk_mixtral_last_hip_error(void);
const char *mk_mixtral_last_error_site(void);
int mk_mixtral_abi_version(void);

#ifdef __cplusplus
}
#endif

#endif /* MK_MIXTRAL_H */
