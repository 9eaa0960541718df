/*
 * hsdpa.h — the C ABI of the MI355X (gfx950) attention step.
 *
 * Drop-in for the full-attention SDPA node of herbert-jit-bf16: decode (one
 * query row against the whole bf16 KV cache) and causal prefill (a chunk of
 * rows with an offset into an existing cache), bf16 q/K/V/out, f32
 * accumulation, GQA head mapping kv_head = q_head / gqa, caller-supplied scale.
 *
 * What each entry point replaces in the reference (paths relative to the
 * reference root):
 *
 *   hsdpa_spec              AttentionSpec, src/jit/execution/abi.rs:136-151,
 *                           plus the cache geometry of KvSpec (abi.rs:57-72)
 *                           and the SdpaShape sink flag (src/jit/ir.rs:55-60)
 *   hsdpa_call              AttentionCall, src/jit/execution/abi.rs:156-180
 *   hsdpa_plan_create       the mount-time pair head_kernel + prefill_kernel
 *                           (src/jit/sdpa.rs:445-512, 111-176) and the
 *                           geometry checks of tile_selector
 *                           (src/jit/target/x86/execution/attention.rs:56-103)
 *   hsdpa_attention         the generated attention node: every task of
 *                           emit_selector (attention.rs:105-224) called by the
 *                           entry loop (src/jit/target/x86/execution/entry.rs:437-483)
 *   hsdpa_status            Decline (src/jit/ir.rs:177-230) and
 *                           ExecutionError (attention.rs:86-98)
 *
 * All strides are in bf16 elements, like the reference. All pointers are
 * device pointers (HBM) except the spec/call/plan structs themselves, which
 * live on the host. Nothing here allocates device memory after
 * hsdpa_plan_create: the caller owns q, the cache, out and the workspace.
 */
#ifndef HSDPA_H
#define HSDPA_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Named refusals. The shape refusals mirror Decline; the others are the
 * run-time checks the reference performs at mount or before entry. */
typedef enum hsdpa_status {
    HSDPA_OK = 0,
    HSDPA_ERR_EMPTY = 1,            /* Decline::Empty: heads, gqa or head_dim is 0 */
    HSDPA_ERR_HEAD_DIM = 2,         /* Decline::HeadDim: not a multiple of 32, above 512,
                                       or above what the GPU kernels hold (256) */
    HSDPA_ERR_GQA = 3,              /* heads not a multiple of gqa (attention.rs:61-64) */
    HSDPA_ERR_STRIDE = 4,           /* q_head < head_dim, heads*q_head > q_row,
                                       heads*head_dim > out_row, kv_stride < capacity*head_dim
                                       (attention.rs:65-75, abi.rs:78-84) */
    HSDPA_ERR_SINK_UNSUPPORTED = 5, /* a softmax sink: never emitted for this model */
    HSDPA_ERR_CAPACITY = 6,         /* past + rows > kv_capacity (model/mounted.rs:634-670) */
    HSDPA_ERR_WORKSPACE = 7,        /* workspace missing or smaller than hsdpa_workspace_bytes */
    HSDPA_ERR_ALIGNMENT = 8,        /* a pointer or stride not 16-byte aligned */
    HSDPA_ERR_NULL = 9,             /* a required pointer is null */
    HSDPA_ERR_HIP = 10,             /* a HIP launch or runtime call failed */
    HSDPA_ERR_NO_DEVICE = 11        /* no gfx950 device current */
} hsdpa_status;

/* Per-layer geometry, fixed at mount (AttentionSpec + cache reserve). */
typedef struct hsdpa_spec {
    uint64_t heads;        /* query heads */
    uint64_t gqa;          /* query heads per KV head */
    uint64_t head_dim;     /* elements per head */
    uint64_t q_row;        /* elements between query rows (2*q_dim on a gated model) */
    uint64_t q_head;       /* elements between query heads */
    uint64_t out_row;      /* elements between output rows */
    uint64_t kv_capacity;  /* positions reserved per KV head */
    uint64_t kv_stride;    /* elements between two KV heads of one cache (>= kv_capacity*head_dim) */
    uint32_t grouped;      /* AttentionSpec::grouped: task order only, no effect on results */
    uint32_t sink;         /* SdpaShape::sink: must be 0 */
} hsdpa_spec;

/* One call of the node (AttentionCall). rows and past are values here: the
 * reference reads them through pointers into its frame at run time. */
typedef struct hsdpa_call {
    const uint16_t *q;       /* token-major: row r, head h at q + r*q_row + h*q_head */
    const uint16_t *keys;    /* head-major cache: head kvh, position p at keys + kvh*kv_stride + p*head_dim */
    const uint16_t *values;  /* same layout as keys */
    uint16_t *output;        /* row r, head h at output + r*out_row + h*head_dim */
    uint64_t rows;           /* rows of this call: 1 = decode, more = causal prefill, 0 = nothing */
    uint64_t past;           /* positions cached before the first row; row r sees past+r+1 keys */
    float scale;             /* 1/sqrt(head_dim) in the engine (src/jit/schedule.rs:189-192) */
    float sink;              /* must be 0 */
    void *workspace;         /* device scratch of at least hsdpa_workspace_bytes() */
    uint64_t workspace_bytes;
} hsdpa_call;

typedef struct hsdpa_plan hsdpa_plan;

/* Validate the geometry and choose the kernels (mount). On success *out
 * receives a plan that stays immutable until hsdpa_plan_destroy. */
hsdpa_status hsdpa_plan_create(const hsdpa_spec *spec, hsdpa_plan **out);

void hsdpa_plan_destroy(hsdpa_plan *plan);

/* Device scratch a call of this plan needs, for any rows and past within
 * kv_capacity. Calls that may run concurrently need distinct workspaces. */
uint64_t hsdpa_workspace_bytes(const hsdpa_plan *plan);

/* The whole attention node: every query head of every row, decode when
 * rows == 1, causal prefill otherwise, enqueued on `stream` (a hipStream_t;
 * NULL is the default stream). Validation happens on the host before any
 * launch; nothing is allocated. */
hsdpa_status hsdpa_attention(const hsdpa_plan *plan, const hsdpa_call *call, void *stream);

/* Static, human-readable name of a status. */
const char *hsdpa_status_string(hsdpa_status status);

/* Library version, MAJOR*10000 + MINOR*100 + PATCH. */
uint32_t hsdpa_version(void);

#ifdef __cplusplus
}
#endif
#endif
