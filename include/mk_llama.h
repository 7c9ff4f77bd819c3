/*
 * mk_llama.h -- C ABI of the dense (Llama) decode VM on the MI355X (gfx950)
 * persistent megakernel.  Exported by the same library as mk_mixtral.h
 * (libmk_mixtral.so); status, error-string and device-query calls are the
 * mk_mixtral_* ones declared there.
 *
 * Replaces the reference's pybind11 binding `mk_llama_3b(...)`
 * (demos/low-latency-llama/llama_3b.cu:26-54), whose argument order is the
 * field order of `llama_3b_globals` (demos/low-latency-llama/llama_3b.cuh)
 * and of the Python caller `interpret_with_mk`
 * (megakernels/demos/latency/mk.py:11-47).  The struct keeps that order;
 * tensors become raw device pointers, and the dimensions the reference
 * compiles in (llama_3b.cuh:20-70) become plain integers.
 *
 * Conventions are those of mk_mixtral.h: bf16 tensors are `uint16_t *`,
 * device pointers on the current HIP device, asynchronous launches on
 * `stream`, the caller zeroes `barriers` before each launch.
 *
 * Instruction queues: `instructions[num_workers][queue_len][32]` int32
 * (megakernels/instructions.py:97-119 layout).  Opcodes
 * (megakernels/demos/latency/instructions.py:32-200):
 *   0 NoOp
 *   1 LayerNorm_QKV_MatVecRopeAppend [1, layer, start_block, end_block]
 *   2 PartialAttention               [2, layer, kv_head, num_partials, partial_idx]
 *   3 AttentionReduction             [3, layer, head_start, num_partials, is_terminal,
 *                                     n, list[n]..., output_partial_idx]
 *   4 O_ProjResidual                 [4, layer, start_block, end_block, reduction_block=0]
 *   5 LayerNormDoubleMatVecSiLU      [5, layer, n, block[n]...]
 *   6 DownProjResidual               [6, layer, start_block, end_block, reduction_block]
 *   7 RMS_LM_Head                    [7, start_block, end_block]
 *
 * Barriers `[bar_layers][bar_ops][bar_width]` int32, counter (layer, opcode)
 * at [layer][opcode-1][idx]; waits proceed once a counter reaches:
 *   opcode 1 waits [l-1][5][0] >= (intermediate / matvec_reduction_size)
 *                                 * (hidden / down_proj_block_size)   (l > 0)
 *   opcode 2 waits [l][0][h] >= head_dim / qkv_block_size for its heads
 *   opcode 3 waits [l][1][head_start] >= num_partials
 *   opcode 4 waits [l][2][0] >= num_attention_heads
 *   opcode 5 waits [l][3][0] >= hidden / o_proj_block_size
 *   opcode 6 waits [l][4][0] >= intermediate / up_gate_proj_block_size
 *   opcode 7 waits [L-1][5][0] as opcode 1
 * and arrive as megakernels/demos/latency/python_vm.py:83-412 does.
 *
 * One deliberate difference from python_vm: opcode 4 reduces over all
 * num_attention_heads * head_dim columns of the O projection, as the
 * reference kernel does (demos/low-latency-llama/matvec_adds.cu:10-36);
 * python_vm's o_proj_residual (latency/python_vm.py:96-117) reduces only the
 * first matvec_reduction_size of them.
 */
#ifndef MK_LLAMA_H
#define MK_LLAMA_H

#include <stdint.h>

#include "mk_mixtral.h"

#ifdef __cplusplus
extern "C" {
#endif

#define MK_LLAMA_ABI_VERSION 3

typedef struct mk_llama_globals {
    uint32_t struct_size;          /* sizeof(mk_llama_globals) */
    uint32_t abi_version;          /* MK_LLAMA_ABI_VERSION */

    /* VM state (llama_3b.cu:33-34) */
    int32_t *barriers;             /* [bar_layers, bar_ops (>= 7), bar_width] */
    int64_t bar_layers, bar_ops, bar_width;
    const int32_t *instructions;   /* [num_workers, queue_len, 32] */
    int64_t num_workers, queue_len;
    int32_t *timings;              /* [num_workers, queue_len, 128] or NULL */

    /* weights (llama_3b.cu:36-42) */
    const uint16_t *qkv_weights;          /* [L, (Hq + 2 Hkv) D, H] */
    const uint16_t *attn_norm_weights;    /* [L, H] */
    const uint16_t *o_weights;            /* [L, H, Hq D] */
    const uint16_t *mlp_norm_weights;     /* [L, H] */
    const uint16_t *up_weights;           /* [L, F, H] */
    const uint16_t *gate_weights;         /* [L, F, H] */
    const uint16_t *down_weights;         /* [L, H, F] */
    const uint16_t *lm_head_norm_weights; /* [H] */
    const uint16_t *lm_head_weights;      /* [V, H] */
    uint16_t *k_cache;                    /* [L, T, Hkv, D] (batch 1) */
    uint16_t *v_cache;                    /* [L, T, Hkv, D] */

    /* rope (llama_3b.cu:44) */
    const float *rope_cos;                /* [>= T, D] fp32, interleaved pairs */
    const float *rope_sin;

    /* activations (llama_3b.cu:46-49) */
    uint16_t *hidden_states;              /* [H], updated in place by opcodes 4 and 6 */
    uint16_t *q_post_rope;                /* [Hq D] */
    uint16_t *attn_out;                   /* [Hq D] */
    float *attn_lse_intermediates;        /* [Hq, P] */
    float *attn_out_intermediates;        /* [Hq, P, D] */
    uint16_t *silu_out;                   /* [F] */
    uint16_t *logits;                     /* [V], written by opcode 7 */

    /* scalars (llama_3b.cu:51-53) */
    uint32_t pos_id;
    float attn_scale;
    float rms_norm_eps;
    int32_t skip_attn_reduction;

    /* dimensions the reference compiles in */
    int32_t num_layers, hidden_size, intermediate_size;
    int32_t num_attention_heads, num_kv_heads, head_dim; /* Hq / Hkv in 1..4 */
    int32_t vocab_size, kv_capacity, attn_partial_slots;

    /* block sizes (latency/scheduler.py:131-141) */
    int32_t up_gate_proj_block_size, down_proj_block_size, o_proj_block_size;
    int32_t qkv_block_size, attn_kv_block_size, lm_head_block_size;
    int32_t matvec_reduction_size; /* column chunk of opcode 6, a multiple of 512 */

    /* optional */
    int32_t *status;               /* NULL: the library's per-device status words */
    uint32_t spin_timeout_us;      /* 0 = 2 s */
    int32_t record_timings;

    /* decode-driver extension (no reference counterpart; the reference's
     * generator runs torch.argmax and the embedding between launches,
     * megakernels/generators.py:121-145), as in mk_mixtral_globals */
    int64_t *argmax_out;                /* argmax of logits when the launch ends, or NULL */
    const uint16_t *next_embed_weights; /* [V, H] bf16 or NULL: hidden_states := row *argmax_out */
    int32_t reset_for_next_launch;      /* nonzero: the barrier tensor is zeroed when the launch ends
                                           (the logits are stored, not accumulated, and need none) */

    /* prefetch switch (no reference counterpart as a field: the reference
     * sets its L2 lookahead at compile time, PREFETCH_LOOKAHEAD in
     * demos/low-latency-llama/matvec_pipeline.cuh:19).  Nonzero: every
     * instruction waits for its inputs before it issues any load, and no
     * weights are staged in LDS for a later instruction; same results.
     * For prefetch on/off comparisons. */
    int32_t late_loads;
} mk_llama_globals;

/* Launch one decode step of the dense VM.  Returns MK_OK or an
 * mk_status_code (host-side validation / HIP failure). */
int mk_llama_launch(const mk_llama_globals *g, void *stream);

/* MK_LLAMA_ABI_VERSION of the library. */
int mk_llama_abi_version(void);

#ifdef __cplusplus
}
#endif

#endif /* MK_LLAMA_H */
