/*
 * dolittle_hip.h -- C ABI of libdlhip.so, the MI355X (gfx950) backend for
 * Dolittle's Qwen3-8B token loop.
 *
 * This is the seam a Dolittle host binds in place of its CUDA backend.  Every
 * entry point is extern "C", takes plain pointers and sizes, and returns an
 * int status (DL_OK or one of the dl_status codes); the message of the last
 * failure on the calling thread is available from dl_last_error().  No HIP,
 * torch or C++ types cross the boundary.
 *
 * Reference interfaces replaced (paths relative to the Dolittle tree):
 *   runtime     gpu::Device / gpu::Queue / buffers      src/gpu/device.h:73-184,
 *               gpu::query_memory                       src/gpu/memory.h:49-56,
 *               gpu::cuda::open_device                  src/gpu/cuda/device.h:29
 *   operations  kernels::cuda::launch_*                 src/kernels/cuda/launch.h:79-109
 *               (the eight-operation catalog of src/kernels/operations.h:169-271)
 *   plan/loop   CachedForwardPlan + DeviceSequence       src/inference/executor.h:242-342,
 *                                                       src/inference/decoding/device.h:84-137
 *   sampling    DeviceCategorical                       src/inference/sampling/device.h:58-85
 *   steering    DeviceIntervention (all-position form)  src/inference/steering/device.h:30-68
 *   capture     DeviceSequence::capture                 src/inference/decoding/device.h:112
 *   injection   EmbeddingOverride                       src/inference/executor.h:129-135,
 *               live Injection + DeviceSequence::replace executor.cpp:1583-1632, decode.cu:221-230
 *   intervention CachedForwardPlan::prepare_intervention src/inference/executor.cpp:1717-1748
 *   NLA vectors DeviceInjection                         src/inference/injection/device.h:29-47,
 *               DeviceDirection, DeviceIntervention     src/inference/steering/device.h:30-68
 *
 * Conventions kept from the reference (src/gpu/device.h:18-25,
 * src/kernels/cuda/launch.h:10-14): launches only enqueue work; they allocate
 * nothing and never wait on the host.  Buffers are borrowed until the queue
 * reaches a later completion point.  Asynchronous device errors surface at
 * the next wait.  Host calls on one device are serialised by the caller.
 */
#ifndef DOLITTLE_HIP_H
#define DOLITTLE_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ------------------------------------------------------------------ status */
/* Mirrors the reference's exception classes (src/gpu/device.h:23-25,
 * src/kernels/operations.h:5-10): invalid_argument, length_error,
 * runtime_error, and a poisoned device after an unrecoverable failure. */
typedef enum dl_status {
  DL_OK = 0,
  DL_INVALID_ARGUMENT = 1,
  DL_LENGTH_ERROR = 2,
  DL_RUNTIME_ERROR = 3,
  DL_POISONED = 4
} dl_status;

/* Message of the last failing call on this thread ("" if none). */
const char* dl_last_error(void);

/* Storage element types (src/tensors/representations/representation.h). */
typedef enum dl_dtype { DL_BF16 = 1, DL_F32 = 2, DL_U32 = 3 /* archive catalogs only */ } dl_dtype;

/* ----------------------------------------------------------------- runtime */
typedef struct dl_device dl_device;
typedef struct dl_queue dl_queue;
typedef struct dl_buffer dl_buffer;
typedef struct dl_event dl_event;

typedef struct dl_device_info {
  char name[64];
  char arch[64];
  uint32_t compute_units;
  uint32_t reserved;
  uint64_t total_bytes;
} dl_device_info;

/* gpu::cuda::open_device (src/gpu/cuda/device.h:29). */
int dl_device_open(int ordinal, dl_device** out);
int dl_device_close(dl_device* device);
/* gpu::Device::info (src/gpu/device.h:138-150). */
int dl_device_info_get(dl_device* device, dl_device_info* out);
/* gpu::query_memory (src/gpu/memory.h:49-56). */
int dl_memory_snapshot(dl_device* device, uint64_t* free_bytes, uint64_t* total_bytes);

/* gpu::Device::allocate (device memory) and allocate_staging (pinned,
 * host-mapped memory) (src/gpu/device.h:150-160). */
int dl_buffer_alloc(dl_device* device, uint64_t bytes, uint64_t alignment, dl_buffer** out);
int dl_staging_alloc(dl_device* device, uint64_t bytes, dl_buffer** out);
int dl_buffer_free(dl_buffer* buffer);
/* Address of the buffer: a device address for device buffers (valid as an
 * operand of the dl_* operations), a host address for staging buffers. */
int dl_buffer_address(dl_buffer* buffer, void** out);
int dl_buffer_size(dl_buffer* buffer, uint64_t* out);

/* gpu::Device::create_queue and gpu::Queue (src/gpu/device.h:160-184). */
int dl_queue_create(dl_device* device, dl_queue** out);
int dl_queue_destroy(dl_queue* queue);
int dl_queue_upload(dl_queue* queue, dl_buffer* dst, uint64_t dst_offset, dl_buffer* src_staging,
                    uint64_t src_offset, uint64_t bytes);
int dl_queue_download(dl_queue* queue, dl_buffer* dst_staging, uint64_t dst_offset, dl_buffer* src,
                      uint64_t src_offset, uint64_t bytes);
int dl_queue_copy(dl_queue* queue, dl_buffer* dst, uint64_t dst_offset, dl_buffer* src,
                  uint64_t src_offset, uint64_t bytes);
/* Convenience transfers from/to pageable host memory; both complete before
 * returning (they wait on the queue). */
int dl_queue_write(dl_queue* queue, dl_buffer* dst, uint64_t dst_offset, const void* host,
                   uint64_t bytes);
int dl_queue_read(dl_queue* queue, void* host, dl_buffer* src, uint64_t src_offset, uint64_t bytes);
/* Ordered copy between two addresses, each a device address (of a
 * dl_buffer, or a device word the library hands out, such as the sampler's
 * result) or the host address of a staging buffer: the transfer the
 * reference's Queue::download / Queue::copy perform on any region, borrowed
 * ones included (src/gpu/device.h:170-172).  Enqueues only. */
int dl_queue_transfer(dl_queue* queue, void* dst, const void* src, uint64_t bytes);
/* Completion points: mark returns a monotonically increasing point; wait
 * blocks until the queue reaches it and reports asynchronous failures. */
int dl_queue_mark(dl_queue* queue, uint64_t* point);
int dl_queue_wait(dl_queue* queue, uint64_t point);
int dl_queue_drain(dl_queue* queue);

/* Timing events recorded on a queue (for measurement only). */
int dl_event_create(dl_device* device, dl_event** out);
int dl_event_destroy(dl_event* event);
int dl_event_record(dl_event* event, dl_queue* queue);
int dl_event_elapsed_ms(dl_event* start, dl_event* stop, float* ms);

/* ----------------------------------------------------- operation catalog */
/* The eight operations of src/kernels/operations.h:169-202, with the launch
 * signatures of src/kernels/cuda/launch.h:79-109.  Operands are device
 * addresses (dl_buffer_address) in the reference's row-major layouts; every
 * result is bit-exact with the reference's numerical contract
 * (docs/architecture/transformer-execution.md:115-170), with this build's
 * deterministic exp/sin/cos/sqrt in place of the unpinned native ones.
 * `device_position`, when non-null, points at a uint64 position in device
 * memory that replaces the host first_position (operations.h:234-239). */

/* launch_projection: Y[R,O] = X[R,I] W[O,I]^T (launch.h:79-82). */
int dl_projection(dl_queue* queue, int dtype, const void* input, const void* weight, void* output,
                  uint64_t rows, uint64_t input_width, uint64_t output_width,
                  const uint64_t* output_position);
/* launch_rms_norm (launch.h:83-85). */
int dl_rms_norm(dl_queue* queue, int dtype, const void* input, const void* weight, void* output,
                uint64_t rows, uint64_t width, float epsilon);
/* launch_rotary (launch.h:86-91). */
int dl_rotary(dl_queue* queue, int dtype, const void* input, void* output, uint64_t positions,
              uint64_t heads, uint64_t width, uint64_t first_position, double theta,
              const uint64_t* device_position, int positioned_output);
/* launch_attention_scale: *output = FP32(1/sqrt(width)) (launch.h:92-93). */
int dl_attention_scale(dl_queue* queue, float* output, uint64_t width);
/* launch_attention (launch.h:94-100): K/V rows [capacity, kv_heads, width]. */
int dl_attention(dl_queue* queue, int dtype, const void* query, const void* key, const void* value,
                 void* output, uint64_t positions, uint64_t query_heads, uint64_t kv_heads,
                 uint64_t width, uint64_t first_position, const uint64_t* device_position,
                 uint64_t capacity, const float* scale);
/* launch_embedding (launch.h:101-103).  `vocabulary` bounds the table: a
 * token id outside it yields a zero row instead of an out-of-bounds read. */
int dl_embedding(dl_queue* queue, int dtype, const uint32_t* tokens, const void* weight,
                 void* output, uint64_t rows, uint64_t width, uint64_t vocabulary);
/* launch_add, launch_silu_multiply (launch.h:104-109). */
int dl_add(dl_queue* queue, int dtype, const void* left, const void* right, void* output,
           uint64_t count);
int dl_silu_multiply(dl_queue* queue, int dtype, const void* gate, const void* up, void* output,
                     uint64_t count);
/* GatherRows (src/kernels/cuda/operations.cpp:544-572): copies the listed
 * rows (host array) of `input` into consecutive rows of `output`. */
int dl_gather_rows(dl_queue* queue, const void* input, void* output, uint64_t row_bytes,
                   const uint64_t* rows, uint64_t count);

/* ------------------------------------------- packed projection fast path */
/* Weight layout is an implementation choice of the backend
 * (docs/architecture/transformer-execution.md:47-48).  The packed layout
 * stores each lane's reduction chain contiguously so that every wavefront
 * load is a contiguous 1 KiB while the reference's partial ownership and
 * merge tree are preserved bit for bit.  Requires BF16, output_width a
 * multiple of 64/P and input_width a multiple of 8P (P from the reference's
 * rule).  The row-major weight is not modified. */
int dl_projection_packed_bytes(uint64_t output_width, uint64_t input_width, uint64_t* bytes);
int dl_projection_pack(dl_queue* queue, const void* weight, void* packed, uint64_t output_width,
                       uint64_t input_width);
int dl_projection_packed(dl_queue* queue, const void* input, const void* packed, void* output,
                         uint64_t rows, uint64_t input_width, uint64_t output_width,
                         const uint64_t* output_position);

/* MFMA projection for many rows (the prefill GEMM): Y[R,O] = X[R,I] W^T
 * with W in the packed layout above, BF16 in and out, FP32 accumulation in
 * MFMA order (tolerance, not bit-exact).  `workspace` holds R*I BF16 for the
 * permuted input.  R and O must be multiples of 128, I a multiple of 8P. */
int dl_prefill_projection(dl_queue* queue, const void* input, const void* packed, void* output,
                          void* workspace, uint64_t rows, uint64_t input_width, uint64_t output_width);

/* Diagnostics of the prefill kernels (tolerance checks, no reference
 * counterpart).  dl_prefill_attention: causal attention of `rows` queries
 * at positions first_position.. over the plan-layout caches (K
 * [kv_heads][capacity][128], V^T [kv_heads*128][capacity]); q_rot is
 * [rows][q_heads*128] after QK norm and RoPE; output rows are in P16
 * order.  dl_prefill_gate_up: SiLU(x Wg^T) * (x Wu^T) for interleaved packed
 * gate/up rows (the resident layout), output rows of `ffn` in P32 order. */
int dl_prefill_attention(dl_queue* queue, const void* q_rot, const void* k_cache, const void* v_cache,
                         void* output, uint64_t rows, uint64_t q_heads, uint64_t kv_heads,
                         uint64_t capacity, uint64_t first_position);
int dl_prefill_gate_up(dl_queue* queue, const void* input, const void* packed, void* output,
                       void* workspace, uint64_t rows, uint64_t hidden, uint64_t ffn);

/* -------------------------------------------------------------- Qwen3 model */
typedef struct dl_qwen3 dl_qwen3;

typedef struct dl_qwen3_config {
  uint32_t layers;          /* 36 */
  uint32_t hidden;          /* 4096 */
  uint32_t q_heads;         /* 32 */
  uint32_t kv_heads;        /* 8 */
  uint32_t head_dim;        /* 128 */
  uint32_t ffn;             /* 12288 */
  uint32_t vocab;           /* 151936 */
  uint32_t tied_embeddings; /* 1: the LM head and the embedding share storage */
  float rms_eps;            /* 1e-6 */
  uint32_t reserved;
  double rope_theta;        /* 1e6 */
} dl_qwen3_config;

/* Parameter roles (src/models/qwen3/checkpoint.cpp:113-149 naming). */
typedef enum dl_qwen3_role {
  DL_ROLE_EMBEDDING = 0,
  DL_ROLE_LM_HEAD = 1,
  DL_ROLE_FINAL_NORM = 2,
  DL_ROLE_INPUT_NORM = 3,
  DL_ROLE_Q = 4,
  DL_ROLE_K = 5,
  DL_ROLE_V = 6,
  DL_ROLE_Q_NORM = 7,
  DL_ROLE_K_NORM = 8,
  DL_ROLE_O = 9,
  DL_ROLE_POST_NORM = 10,
  DL_ROLE_GATE = 11,
  DL_ROLE_UP = 12,
  DL_ROLE_DOWN = 13
} dl_qwen3_role;

/* Allocates resident (packed) storage for every parameter
 * (load_resident_model, src/inference/executor.cpp:772-833). */
int dl_qwen3_create(dl_device* device, dl_queue* queue, const dl_qwen3_config* config,
                    dl_qwen3** out);
int dl_qwen3_destroy(dl_qwen3* model);
/* Seeded synthetic parameters generated on the device: every projection
 * and the embedding ~N(0, weight_std) in BF16, every norm gain 1.0.  Stream
 * ids and the generator are documented in dl_synth.h; element i of the
 * tensor (role, layer) in row-major order uses stream layer*16 + role. */
int dl_qwen3_fill_synthetic(dl_qwen3* model, dl_queue* queue, uint64_t seed, float weight_std);
/* Row-major BF16 transfer of one parameter (packing handled internally). */
int dl_qwen3_write_tensor(dl_qwen3* model, dl_queue* queue, int role, uint32_t layer,
                          const uint16_t* host, uint64_t elements);
int dl_qwen3_read_tensor(dl_qwen3* model, dl_queue* queue, int role, uint32_t layer,
                         uint16_t* host, uint64_t elements);
/* Bytes of resident parameter storage. */
int dl_qwen3_resident_bytes(dl_qwen3* model, uint64_t* bytes);

/* ------------------------------------------------- checkpoint archives */
/* Safetensors archives (src/tensors/formats/safetensors.h:101-117) and the
 * Qwen3 checkpoint binding (src/models/qwen3/checkpoint.h:104-123).  Host
 * code only: these calls touch no GPU.  Malformed or unsupported data is
 * DL_INVALID_ARGUMENT, a limit or overflow DL_LENGTH_ERROR, an I/O or digest
 * mismatch DL_RUNTIME_ERROR.  JSON metadata is read strictly: duplicate keys
 * at any depth, nesting beyond 64 containers, nonfinite numbers and trailing
 * text are rejected. */
typedef struct dl_archive dl_archive;

typedef struct dl_archive_limits { /* safetensors::HeaderLimits */
  uint64_t max_header_bytes;
  uint64_t max_metadata_bytes;
  uint64_t max_tensor_count;
} dl_archive_limits;

typedef struct dl_artifact { /* formats::Artifact: a declared file of the archive */
  const char* relative_path;   /* normalized, relative, inside the root */
  uint64_t byte_size;
  const char* sha256;          /* 64 hex characters */
} dl_artifact;

enum { DL_INTEGRITY_SHA256 = 0, DL_INTEGRITY_PREPARED = 1 };

typedef struct dl_archive_request { /* safetensors::OpenRequest */
  const char* root;
  const char* repository;
  const char* revision;
  const dl_artifact* artifacts;
  const char* const* shards;   /* declared artifacts holding tensors */
  const char* index;           /* declared non-shard index artifact, or null */
  uint64_t max_header_bytes;
  uint64_t max_metadata_bytes;
  uint64_t max_tensor_count;
  uint32_t artifact_count;
  uint32_t shard_count;
  uint32_t verification_workers; /* 1..8 concurrent file hashes */
  int32_t integrity;             /* DL_INTEGRITY_SHA256 or DL_INTEGRITY_PREPARED (sizes only) */
} dl_archive_request;

typedef struct dl_tensor_info {
  const char* name;        /* owned by the archive */
  const uint64_t* shape;   /* owned by the archive; `rank` entries */
  const void* payload;     /* mapped host bytes, or null for a decoded header */
  uint64_t data_offset;    /* within the shard's payload region */
  uint64_t byte_count;
  uint32_t rank;
  int32_t dtype;           /* DL_BF16, DL_F32 or DL_U32 */
} dl_tensor_info;

/* safetensors::parse_header: decodes one header (the JSON alone, without the
 * eight-byte prefix) against a payload region of `data_bytes`: unique names,
 * BF16/F32/U32 types, shapes matching their byte ranges, and a complete,
 * non-overlapping payload partition.  The result is a catalog without
 * payloads, sorted by name; destroy it with dl_archive_destroy. */
int dl_safetensors_parse_header(const char* json, uint64_t json_bytes, uint64_t data_bytes,
                                const dl_archive_limits* limits, dl_archive** out);
/* safetensors::open: maps every declared artifact (sizes checked, SHA-256
 * checked unless DL_INTEGRITY_PREPARED), decodes each shard's header, checks
 * the optional index's weight_map against the shards, and publishes the
 * source identity {repository, revision, artifact digest v1}. */
int dl_safetensors_open(const dl_archive_request* request, dl_archive** out);
int dl_archive_destroy(dl_archive* archive);
int dl_archive_tensor_count(const dl_archive* archive, uint64_t* count);
int dl_archive_tensor_info(const dl_archive* archive, uint64_t index, dl_tensor_info* out);
int dl_archive_find(const dl_archive* archive, const char* name, dl_tensor_info* out);
int dl_archive_identity(const dl_archive* archive, const char** repository, const char** revision,
                        const char** digest);
int dl_archive_artifact(const dl_archive* archive, const char* path, const void** bytes, uint64_t* size);
/* SHA-256 (FIPS 180-4) as 64 lowercase hex characters and a terminator. */
int dl_sha256_hex(const void* data, uint64_t bytes, char* out);

/* qwen3::parse_config (checkpoint.cpp): a Hugging Face Qwen3 config with the
 * actual weight type (DL_BF16 or DL_F32); unknown behavioural settings, tied
 * heads, biases, scaled RoPE and sliding windows are rejected.  `out` gets
 * tied_embeddings 0; context_limit is max_position_embeddings. */
int dl_qwen3_parse_config(const char* json, uint64_t json_bytes, int actual_weight_dtype,
                          uint64_t max_metadata_bytes, dl_qwen3_config* out, uint64_t* context_limit);
/* Serialized tensor name of a role (checkpoint.cpp:113-149). */
int dl_qwen3_tensor_name(int role, uint32_t layer, char* out, uint64_t capacity);
/* qwen3::bind_parameters: the catalog holds exactly the 3 + 11 L tensors of
 * `config`, each with its dense shape and `weight_dtype`. */
int dl_qwen3_bind_parameters(const dl_qwen3_config* config, int weight_dtype, const dl_archive* catalog);
/* qwen3::bind_causal_lm without the upload: the configuration artifact
 * parsed with the first tensor's type, then the parameter binding. */
int dl_qwen3_bind_archive(const dl_archive* archive, const char* configuration_artifact, dl_qwen3_config* out,
                          uint64_t* context_limit, uint64_t* parameter_bytes);
/* Binds `archive` as bind_causal_lm does and uploads every parameter into
 * `model`, whose config must equal the archive's (untied, BF16 weights: no
 * type conversion).  Payloads stream from the mapped shards through bounded
 * pinned staging into the packed resident layout. */
int dl_qwen3_load(dl_qwen3* model, dl_queue* queue, const dl_archive* archive, const char* configuration_artifact);

/* ---------------------------------------------------------------- the plan */
/* A cached forward plan for `batch` (1..8) independent sequences sharing
 * the model, each with a contiguous KV cache of `capacity` (<= 32768)
 * positions.  Every sequence's results are independent of the batch size
 * (transformer-execution.md:180-190): each row keeps the single-row
 * reduction trees. */
typedef struct dl_plan dl_plan;

typedef struct dl_sampling {
  uint32_t mode;      /* 0 greedy, 1 categorical (sampler.h:45-55) */
  uint32_t top_k;     /* 0 disables */
  double temperature; /* > 0 */
  double top_p;       /* (0, 1] */
} dl_sampling;

typedef struct dl_generation_result {
  uint32_t generated; /* tokens produced */
  uint32_t reason;    /* 0 limit, 1 eos/stop id, 2 cancelled, 3 failure (device.h:93) */
  uint32_t status;    /* failure latch (bits): 1 NaN/+inf logit, 2 no finite logit, 4 token outside
                         the vocabulary, 8 invalid injection, 16 invalid intervention */
  uint32_t reserved;
  uint64_t position;  /* next position */
} dl_generation_result;

int dl_plan_create(dl_qwen3* model, dl_queue* queue, uint32_t batch, uint32_t capacity,
                   dl_plan** out);
int dl_plan_destroy(dl_plan* plan);
/* Clears positions and generation state (KV contents are overwritten). */
int dl_plan_reset(dl_plan* plan);
int dl_plan_position(dl_plan* plan, uint64_t* position);

/* Writes cache rows [first_position, first_position + count) of one layer
 * of one sequence from the reference layout [count, kv_heads, head_dim]
 * (keys post-RoPE, values raw), as DeviceSequence cache appends would. */
int dl_plan_write_cache(dl_plan* plan, uint32_t seq, uint32_t layer, uint64_t first_position,
                        uint64_t count, const uint16_t* keys, const uint16_t* values);
/* Reads the same rows back in the reference layout. */
int dl_plan_read_cache(dl_plan* plan, uint32_t seq, uint32_t layer, uint64_t first_position,
                       uint64_t count, uint16_t* keys, uint16_t* values);
/* Device bytes the plan holds (KV caches, scores, row buffers, the prompt
 * passes' scratch once a pass has run; the model's weights are
 * dl_qwen3_resident_bytes). */
int dl_plan_device_bytes(dl_plan* plan, uint64_t* bytes);
/* Moves the plan to `position`: rows below it are treated as cached. */
int dl_plan_seek(dl_plan* plan, uint64_t position);
/* Residual row of sequence `seq` after the last consumed position (the
 * final block output, before the final RMSNorm). */
int dl_plan_read_hidden(dl_plan* plan, uint32_t seq, uint16_t* host);

/* Cached forward of `rows` tokens per sequence at the plan's position
 * (tokens[seq * rows + i]); computes the logits of each sequence's last row.
 * This is the diagnostic chunk path (executor.cpp:932-1031). */
int dl_plan_forward(dl_plan* plan, const uint32_t* tokens, uint32_t rows);
/* BF16 logits [vocab] of sequence `seq` from the last forward or step. */
int dl_plan_read_logits(dl_plan* plan, uint32_t seq, uint16_t* host);
/* Device address of sequence `seq`'s logits row (for dl_sampler_* use). */
int dl_plan_logits_address(dl_plan* plan, uint32_t seq, void** out);

/* Block-output capture (DeviceSequence::capture): after block `layer`'s
 * second residual addition every consumed position's row is copied to
 * capture[seq][position][hidden] (BF16).  layer < 0 disables. */
int dl_plan_set_capture(dl_plan* plan, int32_t layer);
int dl_plan_read_capture(dl_plan* plan, uint32_t seq, uint64_t first_position, uint64_t count,
                         uint16_t* host);
/* All-position residual steering of one sequence: after block `layer`'s
 * output, h <- BF16(FP32(h) + vector[i]) for every position (FP32 vector of
 * `hidden` values).  The capture of that block sees the steered row.  A null
 * vector disables steering for the sequence. */
int dl_plan_set_steering(dl_plan* plan, uint32_t seq, int32_t layer, const float* vector);
/* Embedding override (EmbeddingOverride, executor.h:129-135): the embedding
 * row of absolute prompt position `position` is replaced by `row` (BF16
 * bits) for the sequences in `seq_mask` (bit i = sequence i). */
int dl_plan_set_embedding_override(dl_plan* plan, uint64_t position, const uint16_t* row,
                                   uint32_t seq_mask);
/* Live injection (CachedForwardPlan with Injection::device,
 * executor.cpp:1583-1632; DeviceSequence::replace, decode.cu:221-230):
 * `storage` is a DeviceInjection region (dl_injection_bytes(hidden, DL_BF16)
 * bytes, BF16 output) that the caller keeps alive and submits on the plan's
 * queue before the prompt runs.  Its output row replaces the embedding of
 * prompt position `position` of the sequences in `seq_mask`; a nonzero
 * injection status ends the next generation before it consumes anything,
 * with status bit 8 and reason failure (decode.cu decide_stage).  Replaces
 * any embedding override; a null storage or empty mask removes it. */
int dl_plan_set_injection(dl_plan* plan, uint64_t position, const void* storage, int output_dtype,
                          uint32_t seq_mask);
/* Residual intervention (CachedForwardPlan::prepare_intervention,
 * executor.cpp:1717-1748; DeviceIntervention::submit after the boundary's
 * producer step, executor.cpp:1633-1643): after block `layer`'s output,
 * the row of sequence `seq` at prompt position `position` gets
 * h <- BF16(h + (strength * ||h||) * direction) (steering.cu:107-159).
 * `direction` is `hidden` FP32 values (a DeviceDirection region or host
 * memory), copied at this call.  Every prompt pass (generation from
 * position 0, prefill, forward from position 0) zeroes the plan's
 * [status, count]; a failed application latches status bit 16 and ends the
 * loop, and a loop that finishes with its prompt consumed needs count == 1
 * (decode.cu finish_sequence), else status bit 16 and reason failure.
 * Generation requires position < prompt length.  strength 0, layer < 0 or a
 * null direction removes the intervention; strength must be finite and
 * nonnegative. */
int dl_plan_set_intervention(dl_plan* plan, uint32_t seq, int32_t layer, uint64_t position, const float* direction,
                             float strength);
/* The intervention's device status and application count (the regions of
 * DeviceIntervention::status() and count()). */
int dl_plan_read_intervention(dl_plan* plan, uint32_t* status, uint32_t* count);

/* The prompt pass, replacing the reference's forward of a prompt
 * (executor.cpp:285-716 with the row kernels of projection.cu, attention.cu
 * and normalization.cu): positions [0, prompt_length - 1) in chunks of up to
 * 512 consecutive positions, every row the same reduction chains as a
 * single-position step (the projections of a chunk of 16 rows or more as
 * many-row GEMMs over the same chains).  The caches end bit-identical to
 * consuming the prompt through dl_plan_generate; a following
 * dl_plan_generate with the same prompt resumes at the last prompt position.
 * Capture and steering apply to the prompt positions as in the loop. */
int dl_plan_prefill(dl_plan* plan, const uint32_t* prompt, uint32_t prompt_length);
/* NON-CONFORMING tolerance path (no reference counterpart): the same
 * positions as dl_plan_prefill run as BF16 MFMA GEMMs and causal flash
 * attention (softmax in the reference's order, FP32 exponentials).  The
 * MFMA units accumulate in their own order, so projection outputs differ from
 * the reference chains by one BF16 ulp in about 0.1% of elements; on the
 * synthetic Qwen3-8B model this misses the north-star logits bound and the
 * reference's 36-block budget (scripts/validation/README.md:128-142) by as
 * much as nine one-ulp flips in block 0's cache do.  Use dl_plan_prefill
 * where results must match the reference. */
int dl_plan_prefill_mfma(dl_plan* plan, const uint32_t* prompt, uint32_t prompt_length);
/* Diagnostic: residual-stream rows of the last prefill after its final
 * block (rows [first_row, first_row + count), BF16 [count][hidden]). */
int dl_plan_read_prefill_hidden(dl_plan* plan, uint64_t first_row, uint64_t count, uint16_t* host);
/* Diagnostic: elements [first, first + count) of one prefill row buffer of
 * the last block (0 residual, 1 x in P16 order, 2 x in P32 order, 3 q,
 * 4 k, 5 rotated q, 6 attention output in P16 order, 7 SiLU*up in P32
 * order). */
int dl_plan_read_prefill_buffer(dl_plan* plan, uint32_t which, uint64_t first, uint64_t count,
                                uint16_t* host);

/* Device-owned token loop.  Consumes the prompt (shared by all sequences),
 * then generates up to max_new tokens per sequence with the sampling law of
 * src/inference/sampling/categorical.cpp:146-201 and per-sequence
 * MT19937-64 streams seeded seeds[seq] (null: seed 0).  Stop ids end a
 * sequence after the stop token is emitted.  Work is only enqueued; use
 * dl_plan_collect to wait for and read the results. */
int dl_plan_generate(dl_plan* plan, const uint32_t* prompt, uint32_t prompt_length,
                     uint32_t max_new, const dl_sampling* sampling, const uint64_t* seeds,
                     const uint32_t* stop_ids, uint32_t stop_count);
/* Same as dl_plan_generate but enqueues no step: the caller drives the loop
 * with dl_plan_decode_steps (prompt_length + max_new steps complete it). */
int dl_plan_prepare_generation(dl_plan* plan, const uint32_t* prompt, uint32_t prompt_length,
                               uint32_t max_new, const dl_sampling* sampling,
                               const uint64_t* seeds, const uint32_t* stop_ids,
                               uint32_t stop_count);
/* Enqueues `steps` further decode steps of an active generation (no host
 * wait); used by the benchmark to time steady-state decoding. */
int dl_plan_decode_steps(dl_plan* plan, uint32_t steps);
/* Measurement hooks (not part of the reference interface).  bench_prepare
 * snapshots the live control block into a separate always-active one;
 * launch_kernel then enqueues `count` instances of one decode-step kernel
 * (0 QKV, 1 attention scores, 2 softmax, 3 PV, 4 O + residual, 5 gate/up,
 * 6 down + residual, 7 LM head, 8 short-context fused attention, 10
 * attention + O of one row, 12 QKV + attention + O of one or two rows),
 * cycling
 * through layers from `first_layer`
 * so repeated launches stream distinct weights, on the plan's queue. */
int dl_plan_bench_prepare(dl_plan* plan);
int dl_plan_launch_kernel(dl_plan* plan, uint32_t which, uint32_t first_layer, uint32_t count);
/* Workgroup count of one decode-step kernel at every row count (0: one
 * weight tile per wavefront); re-records the step graph. */
int dl_plan_set_grid(dl_plan* plan, uint32_t which, uint32_t blocks);
/* Waits for the enqueued loop and copies each sequence's generated ids
 * (tokens[seq * max_new + i]) and results. */
int dl_plan_collect(dl_plan* plan, uint32_t* tokens, uint32_t max_new,
                    dl_generation_result* results);
/* Requests cancellation of the running loop (may be called from another
 * thread; DeviceSequence::request_stop, decoding/device.h:126).  The device
 * reads it once per step: a prompt position not yet consumed stays
 * unconsumed; a selected token is still consumed, and nothing further is
 * selected (decode.cu: "a selection promises consumption"). */
int dl_plan_request_stop(dl_plan* plan);

/* DeviceSequence::Event (src/inference/decoding/device.h:86-102), 32 bytes:
 * kind 0 consumed (positions [position, position + count) entered the
 * caches), 1 selected (`token` chosen for absolute position `position`),
 * 2 terminal (status = reason 0 limit / 1 eos / 2 cancelled / 3 failure,
 * position = positions consumed, count = tokens generated, token = the
 * failure status bits), 3 injection (status and norm of the installed
 * DeviceInjection, first when one is installed).  Each sequence of a plan
 * has its own journal, written by the device into pinned host-mapped memory
 * (a system-scope release orders each event before its counter), so events
 * can be read while the loop runs; a generation holds at most
 * prompt + 2 * max_new + 3 events per sequence. */
typedef struct dl_sequence_event {
  uint8_t kind;
  uint8_t reserved[3];
  uint32_t status;
  uint64_t position;
  uint64_t count;
  uint32_t token;
  float norm;
} dl_sequence_event;
/* DeviceSequence::collect (decoding/device.h:136; decode.cu:579-610): event
 * `index` of sequence `seq`.  With wait = 0 the call never blocks: *ready is
 * 1 and *event filled when the event is published, else *ready is 0.  With
 * wait != 0 it polls until the event is published.  Either way a queue that
 * has drained with nothing left to enqueue and without the event, or that
 * has failed, is a DL_RUNTIME_ERROR.  An index beyond the
 * journal's capacity is a DL_LENGTH_ERROR. */
int dl_plan_collect_event(dl_plan* plan, uint32_t seq, uint64_t index, int wait,
                          dl_sequence_event* event, int* ready);
/* Events of sequence `seq` published so far (never blocks). */
int dl_plan_event_count(dl_plan* plan, uint32_t seq, uint64_t* count);
/* Bounded step window (no reference counterpart: HIP graphs have no
 * conditional nodes, so each step of the plan's loop is a host-enqueued
 * graph replay).  steps = n, the default being 16, keeps at most 2n steps
 * enqueued ahead of the device: dl_plan_collect and dl_plan_collect_event
 * enqueue more while the loop is live and none after it stopped, so a
 * stopped loop replays at most 2n idle steps (each a few hundred us on
 * Qwen3-8B).  0 enqueues every step of a generation at once and the loop
 * completes with no further host call; a stop then leaves the remaining
 * steps to replay as no-ops.  A change while a windowed generation still has
 * steps to enqueue is a DL_INVALID_ARGUMENT. */
int dl_plan_set_step_window(dl_plan* plan, uint32_t steps);
/* Diagnostic: steps enqueued since the current generation started. */
int dl_plan_steps_enqueued(dl_plan* plan, uint64_t* steps);

/* ------------------------------------------------------ device sequence */
/* DeviceSequence (src/inference/decoding/device.h:84-137), the autonomous
 * prepared sequence the reference records as one conditional CUDA graph
 * (src/kernels/cuda/decode.cu).  HIP graphs have no conditional nodes, so
 * what the caller submits to the queue between begin and complete is
 * captured into one graph per segment: the set-up before the prompt, the
 * full-chunk prompt body, the remainder body, the first selection, the
 * decode forward, the decode selection tail and the terminal publication.
 * Every decision the CUDA graph's conditional nodes take (repeat the prompt
 * chunk, run the remainder, select, keep decoding) is taken by a device
 * kernel from the same device words at the same point and published to
 * host-mapped memory; a driver thread started by dl_sequence_start launches
 * the segment each decision names, so each body runs exactly as often as
 * the CUDA graph runs it and nothing runs speculatively.  Stages: 0 prefill,
 * 1 tail, 2 first selection, 3 decode.  Events are dl_sequence_event. */
typedef struct dl_sequence dl_sequence;
/* DeviceSequence::device_bytes / host_bytes (device.h:102-103). */
int dl_sequence_device_bytes(uint64_t* bytes);
int dl_sequence_host_bytes(uint64_t prompt, uint64_t generated, uint64_t chunk, uint64_t* bytes);
/* Constructor with its Shape (device.h:91-96). */
int dl_sequence_create(dl_queue* queue, uint64_t prompt, uint64_t generated, uint64_t chunk, int forward_only,
                       dl_sequence** out);
/* Destructor: requests a stop, ends a partial capture, joins the driver and
 * drains the queue before freeing. */
int dl_sequence_destroy(dl_sequence* sequence);
/* DeviceSequence::position (device.h:104): device address of the uint64
 * position that recorded bodies read. */
int dl_sequence_position_address(dl_sequence* sequence, void** out);
/* DeviceSequence::begin (device.h:105-110): device addresses of the
 * sampler's {token, status} and terminal words (null, forward-only), the
 * token-input rows of the recipe, the uploaded prompt, and the optional
 * injection {status, norm} and intervention {status, count} words. */
int dl_sequence_begin(dl_sequence* sequence, const uint32_t* selection, const uint32_t* terminal,
                      uint32_t* token_input, uint64_t token_input_bytes, const uint32_t* prompt,
                      uint64_t prompt_bytes, const uint32_t* injection_status, const float* injection_norm,
                      const uint32_t* intervention_status, const uint32_t* intervention_count);
/* begin_stage / end_stage / begin_selection (device.h:111-114). */
int dl_sequence_begin_stage(dl_sequence* sequence, int stage);
int dl_sequence_end_stage(dl_sequence* sequence);
int dl_sequence_begin_selection(dl_sequence* sequence);
/* capture (device.h:115-116): `rows` rows of `source` copied into the arena
 * `destination` (prompt + generated rows) at the device position. */
int dl_sequence_capture(dl_sequence* sequence, const void* source, uint64_t source_bytes, void* destination,
                        uint64_t destination_bytes, uint64_t row_bytes, uint64_t rows);
/* replace (device.h:117-118): prompt position `marker`'s embedding row
 * replaced by `row` in the body that holds it. */
int dl_sequence_replace(dl_sequence* sequence, const void* row, uint64_t row_bytes, void* embeddings,
                        uint64_t embeddings_bytes, uint64_t marker, uint64_t rows);
/* complete (device.h:119) and prepared_resources (device.h:124). */
int dl_sequence_complete(dl_sequence* sequence);
int dl_sequence_resources(dl_sequence* sequence, uint64_t* device_bytes, uint64_t* host_bytes);
/* start / request_stop / drain (device.h:125-127).  request_stop may run on
 * any thread; drain joins the driver and reports its failure. */
int dl_sequence_start(dl_sequence* sequence);
int dl_sequence_request_stop(dl_sequence* sequence);
int dl_sequence_drain(dl_sequence* sequence);
/* collect (device.h:128; decode.cu:579-600): event `index`.  wait = 0 never
 * blocks (*ready 0 until published); either way a sequence that ended
 * without the event, or whose stream failed, is a DL_RUNTIME_ERROR, and an
 * index past the journal's P + 2G + 2 events a DL_LENGTH_ERROR. */
int dl_sequence_collect(dl_sequence* sequence, uint64_t index, int wait, dl_sequence_event* event, int* ready);
int dl_sequence_event_count(dl_sequence* sequence, uint64_t* count);

/* ------------------------------------------ NLA injection and steering */
/* DeviceInjection (src/inference/injection/device.h:29-47; kernel
 * src/kernels/cuda/injection.cu:49-98; law H2 of
 * docs/architecture/execution-boundary.md:489-498).  storage holds
 * [norm FP32][status uint32][output row]: the row norm is eight strided FP32
 * square sums (separate multiply and add, ascending index) added left to
 * right, then sqrt; out[i] = narrow((h[i] / norm) * scale).  status is 0 on
 * success and 1 if the source or the norm is not finite, the norm is zero or
 * an output overflows; an invalid source writes no output.  The source is
 * never changed.  dl_injection_bytes gives the storage size
 * (DeviceInjection::required_bytes). */
int dl_injection_bytes(uint64_t width, int output_dtype, uint64_t* bytes);
int dl_injection_submit(dl_queue* queue, const void* source, int source_dtype, int output_dtype, uint64_t width,
                        float scale, void* storage);
/* DeviceDirection::submit (src/kernels/cuda/steering.cu:69-100): storage holds
 * [status uint32][uint32][FP32 direction]; the direction is
 * (edited - original) / ||edited - original|| with the same reduction;
 * status 1 (and no direction) for a zero or nonfinite norm. */
int dl_direction_bytes(uint64_t width, uint64_t* bytes);
int dl_direction_submit(dl_queue* queue, const void* original, const void* edited, int dtype, uint64_t width,
                        void* storage);
/* DeviceIntervention (src/kernels/cuda/steering.cu:100-159): state holds
 * [status uint32][count uint32].  initialize zeroes both.  submit updates
 * the row of absolute position `selected` when the residual chunk
 * [rows][width] holds positions [*position, *position + rows) (position is
 * a device uint64): beta = strength * ||h||, h[i] = narrow(h[i] + beta u[i]),
 * count += 1; a second application, a prior failure or a nonfinite value
 * sets status 1 (a row already intervened on is left unchanged). */
int dl_intervention_initialize(dl_queue* queue, uint32_t* state);
int dl_intervention_submit(dl_queue* queue, void* residual, int dtype, uint64_t rows, uint64_t width,
                           const float* direction, const uint64_t* position, uint64_t selected, float strength,
                           uint32_t* state);

/* ------------------------------------------------------- device sampler */
/* DeviceCategorical (src/inference/sampling/device.h:58-85) over one BF16
 * logits row in device memory.  Selection follows the host law of
 * src/inference/sampling/categorical.cpp:146-201 bit for bit: the device
 * decides with guarded FP64 comparisons and replays the serial fold when a
 * decision lies within its error band.  The result is two uint32 words
 * {token, status} (status 0 ok, 1 NaN/+inf logit, 2 no finite logit). */
typedef struct dl_sampler dl_sampler;
/* DeviceCategorical::required_bytes (device.h:69). */
int dl_sampler_required_bytes(uint64_t vocabulary, uint64_t* bytes);
/* Constructor (device.h:60-61): budget below the required bytes is a
 * DL_LENGTH_ERROR; dtype must be DL_BF16 (FP32 rows are rejected). */
int dl_sampler_create(dl_device* device, dl_queue* queue, uint64_t vocabulary, int dtype,
                      uint64_t budget, dl_sampler** out);
int dl_sampler_destroy(dl_sampler* sampler);
/* DeviceCategorical::submit (device.h:70-71): diagnostic selection with
 * explicit draw bits (u = (bits >> 11) * 2^-53); row_bytes = vocabulary * 2. */
int dl_sampler_submit(dl_sampler* sampler, const void* logits, uint64_t row_bytes,
                      const dl_sampling* settings, uint64_t draw_bits);
/* DeviceCategorical::start (device.h:75-76): validates, builds the stop mask
 * and seeds the device MT19937-64 stream once. */
int dl_sampler_start(dl_sampler* sampler, const dl_sampling* settings, uint64_t seed,
                     const uint32_t* stop_ids, uint32_t stop_count);
/* DeviceCategorical::submit_next (device.h:77): one draw from the device
 * stream, then the terminal latch (a stop id or failure freezes the result). */
int dl_sampler_submit_next(dl_sampler* sampler, const void* logits, uint64_t row_bytes);
/* result_storage / terminal_state / current_token (device.h:78-80): device
 * addresses of the 8-byte result, the uint32 terminal latch and the token. */
int dl_sampler_result_address(dl_sampler* sampler, void** out);
int dl_sampler_terminal_address(dl_sampler* sampler, void** out);
int dl_sampler_current_token_address(dl_sampler* sampler, void** out);
/* Waits for the queue and returns {token, status}. */
int dl_sampler_result(dl_sampler* sampler, uint32_t* token, uint32_t* status);
/* Diagnostics without a reference counterpart: always decide by the exact
 * serial replay, and the number of selections the replay decided. */
int dl_sampler_set_exact(dl_sampler* sampler, int exact);
int dl_sampler_exact_replays(dl_sampler* sampler, uint64_t* count);
/* No counterpart in the reference.  The selection of dl_sampler_submit with
 * no sampler object and no allocation, for callers that cannot call
 * hipMalloc (work recorded into a HIP graph, serving loops and harnesses that
 * forbid allocation).  The workspace is a library-owned static device array
 * of 789,760 bytes per GPU (one row's histogram, weights, partials and
 * state), held until the process ends; the caller passes the BF16 logits row
 * (row_bytes = vocabulary * 2, vocabulary at most 2^28, larger is a
 * DL_LENGTH_ERROR) and `result`, device memory for {token, status} written
 * when the queue reaches the call.  Every call on one GPU shares that array:
 * calls that overlap on one GPU (two queues, two threads) race.  Results
 * equal dl_sampler_submit's for the same row, settings and draw bits. */
int dl_sample_noalloc(dl_queue* queue, const void* logits, uint64_t row_bytes, uint64_t vocabulary,
                      const dl_sampling* settings, uint64_t draw_bits, uint32_t* result);

#ifdef __cplusplus
}
#endif

#endif /* DOLITTLE_HIP_H */
