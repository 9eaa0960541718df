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
 *   hsdpa_kv_spec           KvSpec, src/jit/execution/abi.rs:57-73
 *   hsdpa_kv_call           KvCall, src/jit/execution/abi.rs:105-130
 *   hsdpa_kv_check          KvSpec::validate, abi.rs:74-103, and the x86
 *                           refusal of the R16 copies
 *                           (src/jit/target/x86/execution/kv.rs:17-21)
 *   hsdpa_kv_append         the kv-append node (src/jit/schedule/lowering.rs:578-592):
 *                           every task of append
 *                           (src/jit/target/x86/execution/kv.rs:15-69)
 *   hsdpa_head_norm_rope    the head-norm-rope node (lowering.rs:549-577): per row,
 *                           norm_rope (src/jit/target/x86/execution/transforms.rs:32-81)
 *                           around ElemOp::RmsNorm[Gemma] and ElemOp::Rope
 *                           (src/jit/target/x86/emit_elem.rs:239-335, 479-520)
 *   hsdpa_output_gate       the attention-output-gate node (lowering.rs:642-666):
 *                           ElemOp::SigmoidMul per row (emit_elem.rs:350-440)
 *   hsdpa_attention_layer   the attention chain of one layer, lowering.rs:549-666:
 *                           head-norm-rope (q, k), kv-append, attention and
 *                           attention-output-gate in one call and fewer launches
 *   hsdpa_kv_restore        the KV half of Runner::restore_from (src/jit/model.rs:786-856)
 *                           for one layer: snapshot (host) to the live cache (device)
 *   hsdpa_kv_take           the KV half of Runner::snapshot_take (model.rs:728-773)
 *                           for one layer: live cache (device) to the snapshot (host)
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
    HSDPA_ERR_HEAD_DIM = 2,         /* Decline::HeadDim: not a multiple of 32, or above 512
                                       (ir.rs:130-162) */
    HSDPA_ERR_GQA = 3,              /* heads not a multiple of gqa (attention.rs:61-64) */
    HSDPA_ERR_STRIDE = 4,           /* q_head < head_dim, heads*q_head > q_row,
                                       heads*head_dim > out_row, kv_stride < capacity*head_dim
                                       (attention.rs:65-75, abi.rs:78-84) */
    HSDPA_ERR_SINK_UNSUPPORTED = 5, /* spec.sink above 1, or a layer call on a plan with the
                                       sink (the layer's node has none: scheduler.rs:111) */
    HSDPA_ERR_CAPACITY = 6,         /* past + rows > kv_capacity (model/mounted.rs:634-670) */
    HSDPA_ERR_WORKSPACE = 7,        /* workspace missing or smaller than hsdpa_workspace_bytes */
    HSDPA_ERR_ALIGNMENT = 8,        /* a pointer or stride not 16-byte aligned */
    HSDPA_ERR_NULL = 9,             /* a required pointer is null */
    HSDPA_ERR_HIP = 10,             /* a HIP launch or runtime call failed */
    HSDPA_ERR_NO_DEVICE = 11,       /* no gfx950 device current */
    HSDPA_ERR_BATCH = 12,           /* kv append: rows > max_batch (the frame's bound);
                                       attention: rows > the plan's max_rows */
    HSDPA_ERR_LAYOUT = 13,          /* kv append: the R16 copies, an AArch64 layout (kv.rs:19-21) */
    HSDPA_ERR_FORM = 14,            /* an unknown decode form (the knob's parse, knobs.rs:66-68),
                                       or a Fused plan with more than 65 536 query heads per
                                       KV head (more padded decode groups than a grid holds) */
    HSDPA_ERR_STATIC_SCRATCH = 15,  /* hsdpa_attention_static: the plan's workspace exceeds
                                       HSDPA_STATIC_SCRATCH_BYTES */
    HSDPA_ERR_FRAME = 16            /* hsdpa_attention_frame: the plan has no frame route (it needs
                                       max_rows = 1, head_dim 64, 128 or 256, query heads per KV
                                       head in at most 4 equal groups of at most 16, kv_capacity
                                       below 2^31, and decode groups x ceil(kv_capacity / 128)
                                       below 2^31) */
} hsdpa_status;

/* The decode head form (SdpaForm, src/jit/ir.rs:100-115; the knob
 * sdpa_form, src/jit/knobs.rs:66-68). Chained is the reference's default:
 * the exponentials at the row maximum, divided by their sum. Fused is its
 * online softmax over blocks of 16 positions
 * (src/jit/target/x86/emit_sdpa/x86/decode.rs:501-669): each block's
 * exponentials at the running maximum so far, the accumulators rescaled by
 * P(m_old - m_new), the sum's reciprocal at the end. Under Fused, like the
 * reference, the rows the engine serves with its prefill block (full chunks
 * of 8 rows) keep the Chained numerics; the other rows (a decode row, the
 * last rows % 8 of a chunk) take the Fused ones, on the decode kernels
 * whatever the shape (padded groups where no equal split into groups of at
 * most 16 query heads exists); above head_dim 256 the form falls back to
 * Chained (src/jit/sdpa.rs:491-510). */
typedef enum hsdpa_form {
    HSDPA_FORM_CHAINED = 0,
    HSDPA_FORM_FUSED = 1
} hsdpa_form;

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
    uint32_t sink;         /* SdpaShape::sink (ir.rs:55-60): 0, or 1 for the softmax sink of the call's
                              `sink` value: the maximum becomes max(scores, sink), the sum gains
                              exp(sink - max) (decode.rs:239-290); a Fused plan with the sink runs
                              the Chained form, as the engine does when Fused declines it
                              (emit_sdpa.rs:468-470) */
    uint32_t form;         /* hsdpa_form */
    uint32_t reserved;     /* 0 */
    uint64_t max_rows;     /* the most rows one call will pass (0: any, up to kv_capacity); sizes the
                              workspace, like KvSpec::max_batch bounds the frame (abi.rs:57-73):
                              1 gives a decode-only plan with a workspace of a few MiB */
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
    float sink;              /* the sink's score (AttentionCall::sink, abi.rs:174): read when spec.sink is
                                1, ignored otherwise */
    void *workspace;         /* device scratch of at least hsdpa_workspace_bytes() */
    uint64_t workspace_bytes;
} hsdpa_call;

typedef struct hsdpa_plan hsdpa_plan;

/* Validate the geometry and choose the kernels (mount). On success *out
 * receives a plan that stays immutable until hsdpa_plan_destroy. */
hsdpa_status hsdpa_plan_create(const hsdpa_spec *spec, hsdpa_plan **out);

void hsdpa_plan_destroy(hsdpa_plan *plan);

/* Device scratch a call of this plan needs, for any rows (up to max_rows) and
 * past within kv_capacity. Calls that may run concurrently need distinct
 * workspaces. */
uint64_t hsdpa_workspace_bytes(const hsdpa_plan *plan);

/* The kernels a call of `rows` rows after `past` positions would run, without
 * running them (the reference prints its plan under HERBERT_JIT_DEBUG_PLAN,
 * src/jit/sdpa.rs:291-306). A call may take two routes: its leading rows on
 * `main`, its last `tail_rows` rows on `tail` (the Fused form's rows outside
 * full chunks of 8). */
typedef enum hsdpa_kernels {
    HSDPA_KERNELS_NONE = 0,
    HSDPA_KERNELS_DECODE = 1,         /* one row on the decode passes (scores, P.V, combine) */
    HSDPA_KERNELS_FEW_ROWS = 2,       /* a few rows as (row, head) columns of the decode passes */
    HSDPA_KERNELS_CAUSAL = 3,         /* the causal kernel, one workgroup per row group */
    HSDPA_KERNELS_CAUSAL_SPLIT = 4,   /* the causal kernel split over the keys (maxima, P.V, combine) */
    HSDPA_KERNELS_DECODE_ROWS = 5,    /* one decode per row, in turn */
    HSDPA_KERNELS_CAUSAL_SHORT = 6,   /* a short chunk: each 32-row block's keys split among its waves */
    HSDPA_KERNELS_CAUSAL_PAIRED = 7   /* the causal kernel's light and heavy row groups paired (maxima, P.V, combine) */
} hsdpa_kernels;

typedef struct hsdpa_route {
    uint32_t main;          /* hsdpa_kernels of the leading rows */
    uint32_t main_form;     /* hsdpa_form of their numerics */
    uint32_t tail;          /* hsdpa_kernels of the last tail_rows rows (NONE: no tail) */
    uint32_t tail_form;
    uint64_t main_rows, tail_rows;
    uint32_t splits;        /* key splits of CAUSAL_SPLIT, else 1 */
    uint32_t launches;      /* kernel launches of the whole call */
} hsdpa_route;

hsdpa_status hsdpa_attention_route(const hsdpa_plan *plan, uint64_t rows, uint64_t past, hsdpa_route *out);

/* The whole attention node: every query head of every row, the decode kernels
 * when rows == 1 (and for up to 16 rows at head_dim 64, 128 and 256 while
 * rows * gqa <= 128, past 8 rows or 64 columns only over short enough caches),
 * causal prefill otherwise, enqueued on `stream` (a hipStream_t;
 * NULL is the default stream). Validation happens on the host before any
 * launch; nothing is allocated. HSDPA_ERR_HIP after a launch was enqueued
 * leaves the output rows unspecified. */
hsdpa_status hsdpa_attention(const hsdpa_plan *plan, const hsdpa_call *call, void *stream);

/* The attention node without a caller workspace: as hsdpa_attention, with
 * the library's own device scratch in place of call->workspace (the call's
 * workspace and workspace_bytes are ignored). It has no counterpart in the
 * reference; it is for callers that cannot allocate device memory: code under
 * HIP graph capture, tight serving loops, harnesses that forbid hipMalloc.
 * The scratch is one static array of HSDPA_STATIC_SCRATCH_BYTES per GPU,
 * held until the process ends; a plan whose hsdpa_workspace_bytes exceeds it
 * is refused (HSDPA_ERR_STATIC_SCRATCH) before any launch: at 16 query heads on
 * 2 KV heads of head_dim 256 (256 CUs), a decode-only plan (max_rows = 1) fits
 * up to a capacity of 487 424 positions, max_rows = 8 up to 32 512. The call
 * allocates nothing and looks nothing up: hsdpa_plan_create resolves the
 * array's address on the device current at plan creation (a call on a device
 * no plan was created on resolves it there, once). Every call on a GPU shares
 * that GPU's array: calls that overlap on one GPU (different streams, or
 * threads enqueueing at once) race on it; stream-ordered calls do not. */
#define HSDPA_STATIC_SCRATCH_BYTES (32u << 20)
hsdpa_status hsdpa_attention_static(const hsdpa_plan *plan, const hsdpa_call *call, void *stream);

/* ---- A decode step whose rows and past are read at run time ----------------
 * The reference's AttentionCall holds rows and past as pointers into the
 * frame, read by each task when it runs (src/jit/execution/abi.rs:156-180,
 * read at attention.rs:122-130), so that one generated program serves every
 * call. hsdpa_frame_call does the same on the device: *rows and *past are read
 * by the kernels, so one enqueued sequence (or one captured HIP graph) serves
 * successive decode steps as past grows, with nothing re-enqueued on the host.
 * The grids are sized for any past below kv_capacity; the workgroups past the
 * visible keys exit at once.
 *
 * Plans: decode-only (max_rows = 1), head_dim 64, 128 or 256, at most 64
 * query heads per KV head in at most 4 equal groups of at most 16,
 * kv_capacity below 2^31 and kv_heads x groups x ceil(kv_capacity / 128)
 * below 2^31 (the kernels derive each step's configuration in 32-bit
 * arithmetic; otherwise HSDPA_ERR_FRAME); either form. Values read at run time: *rows = 0 computes
 * nothing; *rows = 1 is one decode row with n = *past + 1 keys; *rows > 1 or
 * *past >= kv_capacity compute nothing and report HSDPA_ERR_BATCH or
 * HSDPA_ERR_CAPACITY through *status. The outputs are those of hsdpa_attention
 * on the same values, up to the key partition across workgroups, which here
 * follows n rather than the host's choice. */
typedef struct hsdpa_frame_call {
    const uint16_t *q;        /* as hsdpa_call */
    const uint16_t *keys;
    const uint16_t *values;
    uint16_t *output;
    const uint64_t *rows;     /* device memory, 8-byte aligned: read when the kernels run */
    const uint64_t *past;     /* device memory, 8-byte aligned: read when the kernels run */
    float scale;
    float sink;               /* as hsdpa_call */
    void *workspace;          /* device scratch of at least hsdpa_workspace_bytes() */
    uint64_t workspace_bytes;
    uint32_t *status;         /* device memory or NULL: receives the step's hsdpa_status when it runs */
} hsdpa_frame_call;

/* Enqueue the three decode passes of a frame call on `stream`. Host checks
 * (the plan's frame route, pointers, alignment, workspace) before any launch;
 * the checks of *rows and *past happen on the device. */
hsdpa_status hsdpa_attention_frame(const hsdpa_plan *plan, const hsdpa_frame_call *call, void *stream);

/* ---- KV append: the node before the attention ------------------------------
 * The keys and values of the current block, token-major (row r, KV head h at
 * input + (r*heads + h)*head_dim), copied into the head-major cache at
 * position past + r of head h (cache + h*stride + (past + r)*head_dim). */
typedef struct hsdpa_kv_spec {
    uint64_t heads;        /* KV heads */
    uint64_t head_dim;     /* elements per head */
    uint64_t stride;       /* elements reserved per KV head (>= capacity*head_dim) */
    uint64_t capacity;     /* positions reserved per KV head */
    uint64_t max_batch;    /* maximum rows in one block */
    uint32_t r16;          /* KvSpec::r16: must be 0 */
    uint32_t reserved;     /* 0 */
} hsdpa_kv_spec;

typedef struct hsdpa_kv_call {
    uint16_t *keys;               /* head-major cache */
    uint16_t *values;             /* head-major cache, same layout */
    const uint16_t *input_keys;   /* the block's token-major keys */
    const uint16_t *input_values; /* the block's token-major values */
    uint64_t rows;                /* rows of the block; 0 = nothing */
    uint64_t past;                /* absolute position of the block's first row */
} hsdpa_kv_call;

/* Mount-time validation of the reserve geometry (KvSpec::validate). */
hsdpa_status hsdpa_kv_check(const hsdpa_kv_spec *spec);

/* The append, enqueued on `stream`. Checks the geometry and the call
 * (rows <= max_batch, past + rows <= capacity, non-null pointers) on the host
 * before any launch. Any alignment is accepted; 16-byte aligned pointers with
 * head_dim and stride multiples of 8 take the vector path. */
hsdpa_status hsdpa_kv_append(const hsdpa_kv_spec *spec, const hsdpa_kv_call *call, void *stream);

/* ---- Head RMS norm + RoPE: the node before the KV append ------------------
 * For each row r and head h, x = data + r*row_stride + h*head_stride (head_dim
 * bf16, in place): x <- rmsnorm(x) * w (Gemma: * (1 + w), added in f32), then
 * the rotate_half RoPE on its first rotary_dims dimensions with the pairs
 * (j, j + rotary_dims/2) and the tables' row at position past + r (cos and
 * sin, table_row bf16 apart, rotary_dims/2 used). The engine calls it once
 * for q (q_norm) and once for k (k_norm). */
typedef struct hsdpa_norm_rope_spec {
    uint64_t heads;        /* heads of the buffer (query or KV heads) */
    uint64_t head_dim;     /* a multiple of 32, at most 512 */
    uint64_t head_stride;  /* elements between heads of a row */
    uint64_t row_stride;   /* elements between rows */
    uint64_t rotary_dims;  /* rotated dimensions: a multiple of 32, at most head_dim; 0 = none */
    uint64_t table_row;    /* elements between positions in cos and sin (>= rotary_dims/2) */
    uint64_t positions;    /* positions the tables hold */
    uint32_t plus_one;     /* 1: Gemma convention (1 + w), as Qwen3.5; 0: w */
    uint32_t reserved;     /* 0 */
} hsdpa_norm_rope_spec;

typedef struct hsdpa_norm_rope_call {
    uint16_t *data;          /* q or k, token-major, normalised and rotated in place */
    const uint16_t *weight;  /* head_dim bf16 (q_norm or k_norm) */
    const uint16_t *cos;     /* [positions][table_row] bf16 */
    const uint16_t *sin;     /* same layout */
    uint64_t rows;
    uint64_t past;           /* position of the first row */
    float eps;               /* RMSNorm epsilon */
    float reserved;          /* 0 */
} hsdpa_norm_rope_call;

hsdpa_status hsdpa_head_norm_rope(const hsdpa_norm_rope_spec *spec, const hsdpa_norm_rope_call *call, void *stream);

/* ---- Output gate: the node after the attention ---------------------------
 * attn[r][i] <- attn[r][i] * sigmoid(gate[r][i]) for i < width, computed as
 * attn / (1 + exp(min(-gate, 88))) with the softmax's exponential; on the
 * gated model the gate follows Q on each row of q (gate = q + q_dim,
 * gate_row = q_row). */
typedef struct hsdpa_gate_spec {
    uint64_t width;        /* elements per row (q_dim) */
    uint64_t attn_row;     /* elements between rows of attn */
    uint64_t gate_row;     /* elements between rows of the gate */
} hsdpa_gate_spec;

typedef struct hsdpa_gate_call {
    uint16_t *attn;          /* in place */
    const uint16_t *gate;
    uint64_t rows;
} hsdpa_gate_call;

hsdpa_status hsdpa_output_gate(const hsdpa_gate_spec *spec, const hsdpa_gate_call *call, void *stream);

/* ---- The attention chain of one layer --------------------------------------
 * The nodes the engine emits for a full-attention layer
 * (src/jit/schedule/lowering.rs:549-666): head-norm-rope on q, head-norm-rope on
 * k, kv-append, attention, attention-output-gate. One launch does the two
 * norms and the append (q and k normalised and rotated in place, as the
 * node does; k and v then written into the cache at past .. past+rows-1);
 * the attention follows and applies the gate as it writes the output. Every
 * buffer (q, k, the cache, output) ends bit-identical to hsdpa_head_norm_rope
 * (q), hsdpa_head_norm_rope (k), hsdpa_kv_append, hsdpa_attention and
 * hsdpa_output_gate called in that order with the same arguments. Decode is 4
 * launches instead of 7, prefill 2 instead of 5. The plan gives heads, gqa,
 * head_dim, q_row, q_head, out_row and the cache geometry; the norms take
 * head_dim weights and the RoPE tables as in hsdpa_norm_rope_spec. */
typedef struct hsdpa_layer_call {
    uint16_t *q;              /* [rows][q_row]: each head normalised and rotated in place */
    uint16_t *k;              /* the block's K projections, normalised and rotated in place:
                                 row r, KV head h at k + r*kv_row + h*head_dim */
    const uint16_t *v;        /* the block's V projections, same layout */
    uint16_t *keys;           /* the cache, as hsdpa_call, written at past .. past+rows-1 */
    uint16_t *values;
    uint16_t *output;         /* as hsdpa_call; gated when gate is not null */
    const uint16_t *gate;     /* null: no gate; else row r, head h at gate + r*gate_row + h*head_dim
                                 (q + q_dim with gate_row = q_row on the gated model); 16-byte
                                 aligned, gate_row a multiple of 8 */
    const uint16_t *q_norm;   /* head_dim bf16 */
    const uint16_t *k_norm;   /* head_dim bf16 */
    const uint16_t *cos;      /* [positions][table_row] bf16 (unused when rotary_dims = 0) */
    const uint16_t *sin;
    uint64_t rows;            /* 0 = nothing */
    uint64_t past;
    uint64_t kv_row;          /* elements between rows of k and v (>= kv_heads*head_dim) */
    uint64_t gate_row;
    uint64_t rotary_dims;     /* a multiple of 32, at most head_dim; 0 = none */
    uint64_t table_row;
    uint64_t positions;       /* positions the tables hold */
    float scale;              /* the attention's scale */
    float eps;                /* RMSNorm epsilon */
    uint32_t plus_one;        /* 1: (1 + w), the Gemma convention of Qwen3.5 */
    uint32_t reserved;        /* 0 */
    void *workspace;          /* as hsdpa_call */
    uint64_t workspace_bytes;
} hsdpa_layer_call;

hsdpa_status hsdpa_attention_layer(const hsdpa_plan *plan, const hsdpa_layer_call *call, void *stream);

/* ---- KV snapshot of one layer ----------------------------------------------
 * A snapshot layer holds K[heads][snap_positions][head_dim] then
 * V[heads][snap_positions][head_dim] bf16 (model.rs:675-697), host memory; the
 * live cache is the device layout of hsdpa_kv_spec. `positions` leading
 * positions of every head are copied; positions > snap_positions or >
 * capacity, or a layer block beyond 64 GiB (MAX_BLOCK_SNAPSHOT,
 * model.rs:105-108), is HSDPA_ERR_CAPACITY (snapshot_take's "slot buffer too
 * short" refusal, model.rs:749-755); positions == 0 copies nothing. Enqueued
 * on `stream`; for an asynchronous copy the host buffer must be pinned
 * (hipHostMalloc), pageable memory makes the call return after the copy. */
hsdpa_status hsdpa_kv_restore(const hsdpa_kv_spec *spec, const uint16_t *snapshot_layer, uint64_t snap_positions,
                              uint16_t *keys, uint16_t *values, uint64_t positions, void *stream);
hsdpa_status hsdpa_kv_take(const hsdpa_kv_spec *spec, const uint16_t *keys, const uint16_t *values,
                           uint16_t *snapshot_layer, uint64_t snap_positions, uint64_t positions, void *stream);

/* Static, human-readable name of a status. */
const char *hsdpa_status_string(hsdpa_status status);

/* Library version, MAJOR*10000 + MINOR*100 + PATCH. */
uint32_t hsdpa_version(void);

#ifdef __cplusplus
}
#endif
#endif
