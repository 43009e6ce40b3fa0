/*
 * seeml_hip.h — C-ABI of the MI355X (gfx950) backend for SeeML's compiled
 * LoRA update step.
 *
 * The backend is a drop-in for the reference's op-dispatch seam: it consumes
 * the same .seeu plan bytes (same 64-byte instructions, opcodes, arena
 * offsets decided by the compiler, same load-time validator checks) and
 * executes the train / merge / eval programs on one GPU. All signatures are
 * plain pointers and sizes; no C++ or framework types cross this boundary.
 *
 * Errors: functions return SEEML_HIP_OK (0) or SEEML_HIP_ERROR (1). The
 * message reads "<unit>: <message>" with the reference's unit names
 * ("UpdateEngine", "PlanValidator") — runtime/diagnostics/diagnostic.h:30-41.
 * Engine errors are read with seeml_hip_last_error(); the standalone kernel
 * entry points report through seeml_hip_kernel_error().
 *
 * Threading: one host thread per engine handle; every engine owns one HIP
 * stream, on which all of its work is ordered.
 */
#ifndef SEEML_HIP_H_
#define SEEML_HIP_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define SEEML_HIP_OK 0
#define SEEML_HIP_ERROR 1

/* Program ids: the plan's three instruction streams (schema.h:83-158). */
#define SEEML_HIP_PROGRAM_TRAIN 0
#define SEEML_HIP_PROGRAM_MERGE 1
#define SEEML_HIP_PROGRAM_EVAL 2

typedef struct seeml_hip_engine seeml_hip_engine;

/* ---- Plan integrity and validation (host only; no GPU touched) ----------- */

/* Every load-time proof UpdateEngine::Initialize runs before it allocates
 * (runtime/engine/update_engine.cc:80-225): magic, version window v4..v7,
 * PlanSelfHash seal, VerifyPlanContract (contract.cc:35-100),
 * VerifyExecutorContract incl. ValidateInstruction on every instruction of
 * every program (contract.cc:102-168, plan_validator.cc:9-344), softmax-width
 * and token-plan scans. */
int seeml_hip_verify_plan(const uint8_t* plan, uint64_t plan_size, char* err,
                          uint64_t err_cap);
/* Replaces ValidateInstruction (runtime/validator/plan_validator.h:45-47) for
 * one 64-byte instruction word. */
int seeml_hip_validate_instruction(const void* instr64, uint64_t arena_size,
                                   uint64_t rodata_size, uint32_t plan_version,
                                   char* err, uint64_t err_cap);
/* PlanSelfHash / ContentHash64 (source/identity/hash.h:103-161). */
uint64_t seeml_hip_plan_self_hash(const uint8_t* plan, uint64_t size,
                                  uint64_t hash_offset);
uint64_t seeml_hip_content_hash64(const uint8_t* data, uint64_t size);
/* UpdateEngine::EffectiveLr (update_engine.cc:515-534) for a 280-byte
 * PlanHeader image at `header` and a 1-indexed step. */
float seeml_hip_effective_lr(const uint8_t* header, uint64_t step);

/* ---- Engine lifecycle (replaces UpdateEngine, update_engine.h:119-242) --- */

/* LoadFromMemory + Initialize (update_engine.cc:57-65, 80-276): verifies the
 * plan, then allocates ONE device arena of round64(arena_size) bytes (zeroed,
 * persistent image uploaded) plus a device copy of rodata. The plan bytes
 * are not retained. `device` is the HIP device ordinal. */
int seeml_hip_open(const uint8_t* plan, uint64_t plan_size, int device,
                   seeml_hip_engine** out, char* err, uint64_t err_cap);
void seeml_hip_close(seeml_hip_engine* e);
const char* seeml_hip_last_error(const seeml_hip_engine* e);

/* Decodes a program into its plan-ordered launch list and captures it once
 * as a hipGraph on the engine's stream (replayed by seeml_hip_run).
 * use_graph = 0 selects eager dispatch of the same launch list instead. */
int seeml_hip_build(seeml_hip_engine* e, int program);
int seeml_hip_set_graph_mode(seeml_hip_engine* e, int use_graph);

/* Batch staging into the plan's I/O slots (BatchPipeline::NextBatch,
 * runtime/feeder/batch_pipeline.cc:61-79): input_bytes must equal
 * input_floats*4 and label_bytes the plan's label_bytes. With on_device = 0
 * the buffers are host memory and token ids / class labels are checked
 * against the plan's vocab / class bounds before the copy (the feeder
 * contract, contract.cc:170-235); with on_device = 1 they are device
 * pointers and out-of-range ids poison the loss instead of reading out of
 * bounds. */
int seeml_hip_stage(seeml_hip_engine* e, const void* input, uint64_t input_bytes,
                    const void* labels, uint64_t label_bytes, int on_device);

/* The engine's 1-indexed step_ (AdamW bias correction, LR schedule). Setting
 * it uploads this step's scalars (EffectiveLr, 1/(1-beta^step)). */
int seeml_hip_set_step(seeml_hip_engine* e, uint64_t step);
uint64_t seeml_hip_get_step(const seeml_hip_engine* e);

/* Replays a program (Execute / ExecuteTrainProgram, update_engine.cc:278-304)
 * asynchronously on the engine stream. */
int seeml_hip_run(seeml_hip_engine* e, int program);
/* ExecuteRange (update_engine.cc:306-509): instructions [begin, end) of
 * `program`, each dispatched exactly once, eagerly (no fusion), in plan
 * order on the engine stream. Instruction-by-instruction replay for
 * per-instruction checks and probes. */
int seeml_hip_run_range(seeml_hip_engine* e, int program, uint64_t begin, uint64_t end);
int seeml_hip_sync(seeml_hip_engine* e);
/* LossValue (update_engine.cc:511-513): synchronizes, then reads the f32 at
 * the plan's loss_ref. */
int seeml_hip_loss(seeml_hip_engine* e, float* loss);

/* One iteration of TrainImpl's loop (update_engine.cc:736-753): step_ += 1,
 * scalars, stage, train program, loss read, non-finite abort. */
int seeml_hip_train_step(seeml_hip_engine* e, const void* input, uint64_t input_bytes,
                         const void* labels, uint64_t label_bytes, int on_device,
                         float* loss);

/* RunMerge (update_engine.cc:789-811): the merge program, then a finiteness
 * scan of every emit-table delta. */
int seeml_hip_run_merge(seeml_hip_engine* e);

/* Arena / rodata probes (test/support/probes.cc:25-60; checkpointing of the
 * persistent prefix). `ref` is a plan tensor reference: bit 63 = rodata. */
int seeml_hip_read(seeml_hip_engine* e, uint64_t ref, void* dst, uint64_t bytes);
int seeml_hip_write(seeml_hip_engine* e, uint64_t ref, const void* src, uint64_t bytes);
void* seeml_hip_arena_device_ptr(seeml_hip_engine* e);
void* seeml_hip_stream(seeml_hip_engine* e);
uint64_t seeml_hip_workspace_bytes(const seeml_hip_engine* e);

/* GEMM tile autotuning (compiler/backend/tuner/bandit.cc:14-53,
 * autotuner.cc:21-80 retargeted to GPU tiles): for every distinct GEMM shape
 * of the train program, a deterministic UCB1 bandit over tile arms, reward =
 * measured fraction of fp32 MFMA peak. Every arm keeps the summation order
 * the shape fixes (the split-K count, or the skinny kernels' order): arms
 * differ only in tile config or column split (whole rounds of 256x128 tiles,
 * the rest on smaller tiles), which change no bits, so an autotuned run has
 * the same bits as an untuned one whatever the timings. The pick is the
 * lowest arm within 1.5% of the best mean (arm 0 = the heuristic plan).
 * Picks are installed and graphs rebuilt.
 * budget = launches per shape (at least twice the number of arms). */
int seeml_hip_autotune(seeml_hip_engine* e, int budget);
/* seeml_hip_autotune with injected rewards (the reference's injected reward
 * closure, test/compiler/backend/tuner_test.cc:130-145): each pull's reward
 * is reward(ctx, group, arm, cfg, splits, n_split) for the group-th GEMM
 * shape (in the tuner's order) and its arm-th arm; nothing is launched. */
typedef double (*seeml_hip_tune_reward_fn)(void* ctx, uint64_t group, uint64_t arm, int cfg,
                                           int splits, uint64_t n_split);
int seeml_hip_autotune_injected(seeml_hip_engine* e, int budget, seeml_hip_tune_reward_fn reward,
                                void* ctx);
/* The engine's UCB1 bandit driven like AutotuneGemmTiling
 * (compiler/backend/tuner/autotuner.cc:57-80, bandit.cc:14-53):
 * max(trials, arms) pulls, each rewarded by reward(ctx, arm); picks[t] is
 * the t-th selected arm, pulls/means the per-arm statistics and best_arm
 * BestArm(). Host only. */
typedef double (*seeml_hip_arm_reward_fn)(void* ctx, uint64_t arm);
int seeml_hip_ucb1_run(uint64_t arms, double exploration, uint64_t trials,
                       seeml_hip_arm_reward_fn reward, void* ctx, uint64_t* picks,
                       uint64_t* pulls, double* means, uint64_t* best_arm);
/* Profiling support, no reference counterpart: the algorithmic work of
 * what instruction `index`'s row carries in seeml_hip_profile_program's
 * breakdown where the fused graph launches it differently from the lone
 * instruction — a colsum group's one pass over its shared operand (the
 * large operand counted once; an earlier member's operand copy as bytes
 * only), a dual pass, a LoRA run's base GEMM with its epilogue and the
 * rowdots it launches, a dense GEMM with its fused AddEW. *flops and
 * *bytes are -1 where the instruction's own work applies. Fusions are
 * planned when the program's graph is built. */
int seeml_hip_launch_work(seeml_hip_engine* e, int program, uint64_t index, double* flops,
                          double* bytes);
/* Describe the kernel variant chosen for instruction `index` of `program`:
 * GEMMs "cfg-name splits=S" (or "skinny/<kind>"; a column split reads
 * "cfg|tail-cfg@n_split splits=1"), with " +AddEW" when the
 * AddEW after it runs in its epilogue (that AddEW then reads "in GEMM
 * epilogue"); SoftmaxRowsBwd "causal S=n" when its probabilities are proven
 * AttnFwd/AttnDP outputs (only their causal half is read), else ""; AttnFwd,
 * AttnDP and a causal SoftmaxRowsBwd add "no zero tail" when no reader looks
 * past the diagonal tiles (those zeros are not stored), AttnFwd "P unused"
 * when P has no reader; other opcodes "". Fusions are planned when the
 * program's graph is built. */
int seeml_hip_gemm_choice(seeml_hip_engine* e, int program, uint64_t index, char* buf,
                          uint64_t cap);
/* Test hook: forces instruction `index`'s GEMM plan to tile config `cfg`
 * (seeml_hip_gemm_config_count() - 1 is the skinny kernels) with `splits`
 * slices; the program's graph and fusions are re-planned on its next run. */
int seeml_hip_set_gemm_plan(seeml_hip_engine* e, int program, uint64_t index, int cfg, int splits);

/* ---- Feeder (replaces runtime/feeder/dataset.h:39-177) --------------------
 * A host dataset of fixed-shape samples: feature rows (f32) with class (i32)
 * or dense (f32) labels, or token records of seq+1 i32 ids whose inputs are
 * tokens[0..S) and labels the shifted view tokens[1..S]. Served sequentially
 * with wraparound, or through a seeded splitmix64 Fisher-Yates permutation
 * re-drawn every epoch; the served bytes and order are the reference's.
 * Errors read "Dataset: <message>" (runtime/diagnostics/feeding/error.h). */
typedef struct seeml_hip_dataset seeml_hip_dataset;
/* splitmix64 step (dataset.cc:344-352). */
uint64_t seeml_hip_splitmix64(uint64_t* state);
/* Dataset::FromTokens / FromMemory / LoadFromFile (dataset.cc:34-197). */
int seeml_hip_dataset_from_tokens(const int32_t* tokens, uint64_t count, uint64_t num_records,
                                  uint64_t seq, seeml_hip_dataset** out, char* err,
                                  uint64_t err_cap);
int seeml_hip_dataset_from_memory(const float* inputs, uint64_t input_count,
                                  const uint8_t* labels, uint64_t label_bytes,
                                  uint64_t num_samples, uint64_t input_dim, uint32_t label_kind,
                                  uint64_t label_dim, seeml_hip_dataset** out, char* err,
                                  uint64_t err_cap);
int seeml_hip_dataset_load(const char* path, seeml_hip_dataset** out, char* err,
                           uint64_t err_cap);
/* Dataset::SaveToFile (dataset.cc:230-286), the .sds bytes. */
int seeml_hip_dataset_save(seeml_hip_dataset* d, const char* path);
void seeml_hip_dataset_free(seeml_hip_dataset* d);
const char* seeml_hip_dataset_error(const seeml_hip_dataset* d);
uint64_t seeml_hip_dataset_num_samples(const seeml_hip_dataset* d);
uint64_t seeml_hip_dataset_input_dim(const seeml_hip_dataset* d);
uint32_t seeml_hip_dataset_label_kind(const seeml_hip_dataset* d);
uint32_t seeml_hip_dataset_input_kind(const seeml_hip_dataset* d);
uint64_t seeml_hip_dataset_label_bytes_per_sample(const seeml_hip_dataset* d);
/* Dataset::ValidateClassLabels (dataset.cc:199-228). */
int seeml_hip_dataset_validate_class_labels(seeml_hip_dataset* d, uint64_t num_classes);
/* Dataset::FillBatch (dataset.cc:288-342) into HOST slots: token corpora
 * take `batch` token rows (a whole number of records). */
void seeml_hip_dataset_fill_batch(seeml_hip_dataset* d, uint64_t batch, void* input_slot,
                                  void* label_slot);
/* Rewind / EnableShuffle / SaveServingPos / RestoreServingPos / SkipServed /
 * SplitValidation (dataset.h:95-150, dataset.cc:356-462). */
void seeml_hip_dataset_rewind(seeml_hip_dataset* d);
void seeml_hip_dataset_enable_shuffle(seeml_hip_dataset* d, uint64_t seed);
void seeml_hip_dataset_get_serving_pos(const seeml_hip_dataset* d, uint64_t* cursor,
                                       uint64_t* epoch);
void seeml_hip_dataset_restore_serving_pos(seeml_hip_dataset* d, uint64_t cursor,
                                           uint64_t epoch);
int seeml_hip_dataset_skip_served(seeml_hip_dataset* d, uint64_t rows);
int seeml_hip_dataset_split_validation(seeml_hip_dataset* d, double fraction,
                                       seeml_hip_dataset** val);

/* ---- Train / evaluate loops (UpdateEngine::Train / EvaluateMetrics) -------
 * The engine drives the feeder itself: a host thread fills the next batch
 * into pinned memory while the current step runs, and each step's batch is
 * one H2D copy per I/O slot on the engine stream (batch_pipeline.cc). */
typedef struct seeml_hip_eval_metrics {
  float loss;           /* mean of per-batch eval losses, in double */
  int32_t has_accuracy; /* class-label plan whose eval softmax covers the batch */
  float accuracy;       /* strict-'>' argmax hits / real (unwrapped) rows */
} seeml_hip_eval_metrics;
typedef struct seeml_hip_train_report { /* TrainReport, update_engine.h:91-117 */
  uint64_t steps;
  float initial_avg_loss;
  float final_avg_loss;
  int32_t has_validation;
  float val_initial_loss;
  float val_final_loss;
  int32_t has_val_accuracy;
  float val_initial_accuracy;
  float val_final_accuracy;
  int32_t improved; /* TrainReport::improved(): the regression gate */
  int32_t stopped_early; /* should_stop interrupted the run (update_engine.h:93) */
} seeml_hip_train_report;
/* EvaluateMetrics (update_engine.cc:557-650): snapshot + rewind the set, the
 * eval program per compiled batch (the last batch wraps), loss mean in
 * double, accuracy on device over the real rows, serving position restored. */
int seeml_hip_evaluate_metrics(seeml_hip_engine* e, seeml_hip_dataset* d,
                               seeml_hip_eval_metrics* out);
/* TrainImpl (update_engine.cc:664-787): validation before/after when given,
 * `steps` (0 = the plan's default_steps) train steps from the engine's
 * step_, non-finite loss aborts, first/last-window loss means; loss_curve
 * (optional) receives up to curve_cap per-step losses. */
int seeml_hip_train(seeml_hip_engine* e, seeml_hip_dataset* d, uint64_t steps,
                    seeml_hip_dataset* validation, float* loss_curve, uint64_t curve_cap,
                    seeml_hip_train_report* out);

/* TrainOptions (update_engine.h:40-60): with checkpoint_path and
 * checkpoint_every > 0, a checkpoint is saved whenever step_ is a multiple
 * of checkpoint_every; with resume, checkpoint_path is loaded first (a
 * missing or unusable one is reported on stderr and training starts from
 * the current state) and the feeder skips the step_ * batch rows already
 * served, so a resumed run is the uninterrupted one bit for bit
 * (update_engine.cc:676-696, 766-770). should_stop (may be NULL) is
 * TrainOptions::should_stop, polled once before each step on the calling
 * thread; a nonzero return ends the run there with report.stopped_early
 * set and report.steps the steps executed (update_engine.cc:737-740). With
 * checkpointing, a stopped run resumes where it stopped. */
typedef int (*seeml_hip_should_stop_fn)(void* ctx);
typedef struct seeml_hip_train_options {
  const char* checkpoint_path; /* NULL or "": no checkpointing */
  uint64_t checkpoint_every;   /* steps between checkpoints; 0 = off */
  int32_t resume;
  seeml_hip_should_stop_fn should_stop; /* NULL: never stop early */
  void* should_stop_ctx;
} seeml_hip_train_options;
/* seeml_hip_train with TrainOptions (options may be NULL). */
int seeml_hip_train_ex(seeml_hip_engine* e, seeml_hip_dataset* d, uint64_t steps,
                       seeml_hip_dataset* validation, float* loss_curve, uint64_t curve_cap,
                       const seeml_hip_train_options* options, seeml_hip_train_report* out);

/* SaveCheckpoint / LoadCheckpoint (update_engine.cc:894-913): the arena's
 * persistent segment and step_ in the SEKP container
 * (runtime/custodian/checkpoint.h:8-24): u32 "SEKP", u32 version 3,
 * u64 plan_hash, u64 step, u64 persistent_size, u64 ContentHash64 of the
 * payload, then the payload. Saves are durable (temporary file, fsync,
 * rename, directory fsync); loads verify magic, version, plan binding, size
 * and payload hash before any byte reaches the arena, then set step_.
 * Errors read "Checkpoint: <message>". */
int seeml_hip_save_checkpoint(seeml_hip_engine* e, const char* path);
int seeml_hip_load_checkpoint(seeml_hip_engine* e, const char* path);
/* The container alone, host only (SaveCheckpointFile / LoadCheckpointFile,
 * checkpoint.cc:39-83): read copies the verified payload (exactly `size`
 * bytes) into dst and the saved step into *step; dst is untouched on error. */
int seeml_hip_checkpoint_write(const char* path, uint64_t plan_hash, uint64_t step,
                               const uint8_t* payload, uint64_t size, char* err, uint64_t err_cap);
int seeml_hip_checkpoint_read(const char* path, uint64_t plan_hash, uint64_t size, uint8_t* dst,
                              uint64_t* step, char* err, uint64_t err_cap);

/* Profiling (outside any timed step): replays `program` eagerly `reps`
 * times on the engine stream with a HIP event pair around every
 * instruction, and writes each instruction's mean duration in ms to
 * ms_out[count] (count = the program's instruction count). The program's
 * side effects happen `reps` times (optimizer state moves). */
int seeml_hip_profile_program(seeml_hip_engine* e, int program, int reps, float* ms_out,
                              uint64_t count);
/* Timing inside ordinary replays: the launches of `indices` (a marked tile
 * group's first instruction times the whole group launch) run between two
 * wall-clock stamp nodes of the program's one graph (rebuilt on next run),
 * which accumulate each launch's time on the device.
 * seeml_hip_marked_times returns each marked launch's mean duration (ms)
 * over the replays since the marks were set or last read, in ascending
 * index order, and restarts the sums. Without a graph (or a device wall
 * clock), HIP events around each marked launch give the latest replay's
 * duration. Marked instructions are left out of the other fusions.
 * count = 0 removes the marks. */
int seeml_hip_mark_timed(seeml_hip_engine* e, int program, const uint64_t* indices,
                         uint64_t count);
int seeml_hip_marked_times(seeml_hip_engine* e, int program, float* ms_out, uint64_t count);
/* Mean duration (ms) of one instruction's launch sequence, relaunched
 * `reps` times between two events on the engine stream. */
int seeml_hip_time_instruction(seeml_hip_engine* e, int program, uint64_t index, int reps,
                               float* avg_ms);
uint64_t seeml_hip_program_length(const seeml_hip_engine* e, int program);

/* ---- Standalone kernels (update_kernels.h:27-162 on device pointers) ------
 * Same argument meaning as the reference kernels; `stream` is a hipStream_t
 * (NULL = default stream). Scratch comes from a library-owned per-device
 * workspace; calls on one device must not overlap. */
const char* seeml_hip_kernel_error(void);
int seeml_hip_gemm_nn(const float* A, const float* B, float* C, uint64_t M, uint64_t N,
                      uint64_t K, const float* bias, int act, void* stream);
int seeml_hip_gemm_nt(const float* A, const float* B, float* C, uint64_t M, uint64_t N,
                      uint64_t K, void* stream);
int seeml_hip_gemm_tn(const float* A, const float* B, float* C, uint64_t M, uint64_t N,
                      uint64_t K, void* stream);
/* seeml_hip_gemm_tn without allocation. No counterpart in the reference: it
 * is for callers that cannot allocate device memory (code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc). Same plan,
 * kernels and bits as seeml_hip_gemm_tn, but its scratch is a fixed device
 * array of SEEML_HIP_NOALLOC_SCRATCH_BYTES per GPU, held until the process
 * ends; a shape needing more is rejected with an error before any launch.
 * It calls no hipMalloc/hipFree. Calls that overlap on one GPU race on the
 * shared array. */
#define SEEML_HIP_NOALLOC_SCRATCH_BYTES (16u << 20)
int seeml_hip_gemm_tn_noalloc(const float* A, const float* B, float* C, uint64_t M, uint64_t N,
                              uint64_t K, void* stream);
int seeml_hip_gemm_acc_nn(const float* A, const float* B, float* C, uint64_t M, uint64_t N,
                          uint64_t K, float alpha, void* stream);
int seeml_hip_gemm_nn_q8(const float* A, const int8_t* B, float* C, uint64_t M, uint64_t N,
                         uint64_t K, float scale, int act, void* stream);
int seeml_hip_gemm_nt_q8(const float* A, const int8_t* B, float* C, uint64_t M, uint64_t N,
                         uint64_t K, float scale, void* stream);
/* GEMM with an explicit tile config / split count (autotuner arms, tests). */
int seeml_hip_gemm_forced(int layout, const float* A, const float* B, float* C, uint64_t M,
                          uint64_t N, uint64_t K, int cfg, int splits, void* stream);
/* The LoRA backward's two GEMMs over one stream x [T, D] in one pass (the
 * engine fuses the plan's adjacent pair; tests call it directly): dt = x b^T
 * (b [r_rd, D]) and db = t^T x (t [T, r_cs]), ranks <= 16, x scaled by
 * `scale` as loaded when `scaled`. which: 1 = dt only, 2 = db only, 3 =
 * both; each output has the same bits in every form. No reference
 * counterpart: the reference runs the two GEMMs (gemm.cc:173-200). */
int seeml_hip_gemm_skinny_dual(const float* x, uint64_t T, uint64_t D, const float* b,
                               uint64_t r_rd, float* dt, const float* t, uint64_t r_cs, float* db,
                               int which, int scaled, float scale, void* stream);
/* The q/k/v LoRA GEMMs over one layer input x [T, D] as one pass over x
 * (the engine groups the plan's members; tests call it directly), n = 2..4
 * members of rank r <= 16. kind 0, the rowdot group: out[j] = x a[j]
 * (a[j] [D, r] row-major, out[j] [T, r]). kind 1, the colsum group:
 * out[j] = x^T a[j] (a[j] [T, r], out[j] [D, r]). Each output has the bits
 * of its own skinny GEMM. No reference counterpart: the reference runs each
 * GEMM on its own (gemm.cc:173-200). */
int seeml_hip_gemm_skinny_group(int kind, const float* x, uint64_t T, uint64_t D,
                                const float* const* a, uint64_t r, float* const* out, int n,
                                void* stream);
/* GEMMs as one tile-group launch (the engine groups a plan's consecutive
 * independent GEMM launches; tests call it directly): n = 2..4 members of
 * one layout (0 NN, 1 NT), all on tile config `cfg`; member j is C[j] =
 * A[j] B[j] of shape (M, N, K) = dims[3j .. 3j + 2], and with addend[j] set
 * (addend may be null), the fused AddEW out[j] = addend[j] + C[j] with C[j]
 * not stored. Each output has the bits of its member's own launch. No
 * reference counterpart: the reference runs each GEMM on its own
 * (gemm.cc:173-200). */
int seeml_hip_gemm_group(int layout, int cfg, int n, const float* const* A, const float* const* B,
                         float* const* C, const uint64_t* dims, const float* const* addend,
                         float* const* out, void* stream);
/* GEMM as two launches over column ranges (tests): columns [0, n_split) on
 * tile config `cfg`, the rest on `tail_cfg` (both one split); with `out`,
 * the fused AddEW out = addend + C, and C not stored when C is null.
 * n_split = 0: one launch of `cfg`. */
int seeml_hip_gemm_forced_split(int layout, const float* A, const float* B, float* C, uint64_t M,
                                uint64_t N, uint64_t K, int cfg, int tail_cfg, uint64_t n_split,
                                const float* addend, float* out, void* stream);
/* GEMM (NN or NT, tile config `cfg`: 2, or 0 for NT) with a LoRA
 * up-projection in its epilogue (tests): out = y (+) s where y = A B,
 * u = t bl (t [M, r] row-major, bl [r, N] row-major, r = 8 or 16, in
 * the k order of a tile GEMM), s = scale * u when `scaled` (else u), and
 * y_first selects the sum's operand order. Only `out` is written. With
 * n_split > 0 the GEMM runs as a column split: [0, n_split) on `cfg`, the
 * rest on `tail_cfg` (bl's columns offset like B's). */
int seeml_hip_gemm_forced_lora(int layout, const float* A, const float* B, float* out, uint64_t M,
                               uint64_t N, uint64_t K, int cfg, int tail_cfg, uint64_t n_split,
                               const float* t, const float* bl, uint64_t r, int scaled,
                               float scale, int y_first, void* stream);
/* GEMM with a Scale folded into its streamed operand's loads (tests): C =
 * A B with the stream read as fl(scale * x), on tile config `cfg` with
 * `splits` split-K slices. layout 1: NT rowdot shape (N <= 64, A the
 * stream); layout 2: TN colsum shape with M <= 64 (B the stream). Same bits
 * as a Scale into a buffer, then the GEMM on that plan. No reference
 * counterpart: the reference runs the Scale and the GEMM (gemm.cc:173-200). */
int seeml_hip_gemm_forced_scaled(int layout, const float* A, const float* B, float* C, uint64_t M,
                                 uint64_t N, uint64_t K, int cfg, int splits, float scale,
                                 void* stream);
int seeml_hip_gemm_config_count(void);
/* Name of tile config `cfg` ("MTMxMTNxKT/wWMxWN"), "?" when out of range. */
const char* seeml_hip_gemm_config_name(int cfg);

int seeml_hip_add_ew(const float* x, const float* y, float* out, uint64_t n, void* stream);
int seeml_hip_mul_ew(const float* x, const float* y, float* out, uint64_t n, void* stream);
int seeml_hip_add_bias(const float* x, const float* b, float* out, uint64_t rows, uint64_t cols,
                       void* stream);
int seeml_hip_scale(const float* x, float* out, float alpha, uint64_t n, void* stream);
int seeml_hip_reduce_rows(const float* dy, float* db, uint64_t rows, uint64_t cols, void* stream);
int seeml_hip_relu_fwd(const float* x, float* out, uint64_t n, void* stream);
int seeml_hip_relu_bwd(const float* dy, const float* x, float* dx, uint64_t n, void* stream);
int seeml_hip_gelu_fwd(const float* x, float* out, uint64_t n, void* stream);
int seeml_hip_gelu_bwd(const float* dy, const float* x, float* dx, uint64_t n, void* stream);
int seeml_hip_silu_fwd(const float* x, float* out, uint64_t n, void* stream);
int seeml_hip_silu_bwd(const float* dy, const float* x, float* dx, uint64_t n, void* stream);
int seeml_hip_embed_fwd(const int32_t* tokens, const float* table, float* out, uint64_t rows,
                        uint64_t dim, uint64_t vocab, void* stream);
int seeml_hip_fill(float* dst, float value, uint64_t n, void* stream);
int seeml_hip_copy(const float* src, float* dst, uint64_t n, void* stream);
int seeml_hip_layer_norm_fwd(const float* x, const float* gamma, const float* beta, float* y,
                             float* mean, float* rstd, uint64_t rows, uint64_t cols, void* stream);
int seeml_hip_layer_norm_bwd(const float* dy, const float* x, const float* gamma,
                             const float* mean, const float* rstd, float* dx, uint64_t rows,
                             uint64_t cols, void* stream);
int seeml_hip_rms_norm_fwd(const float* x, const float* gamma, float* y, float* rstd,
                           uint64_t rows, uint64_t cols, void* stream);
int seeml_hip_rms_norm_bwd(const float* dy, const float* x, const float* gamma,
                           const float* rstd, float* dx, uint64_t rows, uint64_t cols,
                           void* stream);
int seeml_hip_rope_fwd(const float* x, float* y, uint64_t B, uint64_t S, uint64_t H, uint64_t d,
                       float base, void* stream);
int seeml_hip_rope_bwd(const float* dy, float* dx, uint64_t B, uint64_t S, uint64_t H, uint64_t d,
                       float base, void* stream);
int seeml_hip_attn_fwd(const float* q, const float* k, const float* v, float* o, float* probs,
                       uint64_t B, uint64_t S, uint64_t H, uint64_t d, void* stream);
int seeml_hip_attn_dp(const float* dout, const float* v, float* dp, uint64_t B, uint64_t S,
                      uint64_t H, uint64_t d, void* stream);
int seeml_hip_attn_dv(const float* probs, const float* dout, float* dv, uint64_t B, uint64_t S,
                      uint64_t H, uint64_t d, void* stream);
int seeml_hip_softmax_rows_bwd(const float* probs, const float* dp, float* ds, uint64_t rows,
                               uint64_t cols, void* stream);
int seeml_hip_attn_dq(const float* ds, const float* k, float* dq, uint64_t B, uint64_t S,
                      uint64_t H, uint64_t d, void* stream);
int seeml_hip_attn_dk(const float* ds, const float* q, float* dk, uint64_t B, uint64_t S,
                      uint64_t H, uint64_t d, void* stream);
int seeml_hip_softmax_xent_fwd(const float* logits, const int32_t* labels, float* loss,
                               float* probs, uint64_t N, uint64_t C, void* stream);
int seeml_hip_softmax_xent_bwd(const float* probs, const int32_t* labels, const float* seed,
                               float* dlogits, uint64_t N, uint64_t C, void* stream);
/* EvaluateMetrics' accuracy count (update_engine.cc:619-633) on device
 * pointers: rows whose first strict-'>' argmax equals a non-negative label. */
int seeml_hip_argmax_correct(const float* probs, const int32_t* labels, uint64_t rows,
                             uint64_t cols, uint64_t* correct, void* stream);
int seeml_hip_mse_fwd(const float* pred, const float* target, float* loss, uint64_t n,
                      void* stream);
int seeml_hip_mse_bwd(const float* pred, const float* target, const float* seed, float* dpred,
                      uint64_t n, void* stream);
int seeml_hip_kl_distill_fwd(const float* s_logits, const float* t_logits, float* loss,
                             float* p_s, float* p_t, uint64_t N, uint64_t C, float T,
                             void* stream);
int seeml_hip_kl_distill_bwd(const float* p_s, const float* p_t, const float* seed,
                             float* dlogits, uint64_t N, uint64_t C, float T, void* stream);
int seeml_hip_clip_norm(float* g, uint64_t n, float max_norm, void* stream);
int seeml_hip_sgd_step(float* p, const float* g, uint64_t n, float lr, float weight_decay,
                       void* stream);
int seeml_hip_adamw_step(float* p, const float* g, float* m, float* v, uint64_t n, float lr,
                         float beta1, float beta2, float eps, float weight_decay, uint64_t step,
                         void* stream);

#ifdef __cplusplus
}
#endif

#endif /* SEEML_HIP_H_ */
