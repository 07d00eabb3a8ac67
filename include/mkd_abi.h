/*
 * mkd_abi.h -- C ABI of the MI355X Qwen3-0.6B decode-step library
 * (libmkd_decode.so, built from decode-fusion-boundary_amd/csrc).
 *
 * Plain pointers, sizes and PODs only: no torch or HIP types appear in a
 * signature (streams are passed as `void*` holding a hipStream_t). Every entry
 * point returns 0 on success or a negative MKD_E* code; mkd_last_error()
 * returns the message of the calling thread's last failure.
 *
 * Reference interfaces these replace (tmchao7/decode-fusion-boundary):
 *   MkdStepDesc           <- tg::TgLaunchDesc, tg_abi.h:118-183
 *   mkd_launch_persistent <- extern "C" tg_launch_decode(const TgLaunchDesc*,
 *                            cudaStream_t), taskgraph_kernel.cu:1927-1987
 *                            (bound as nanovllm_megakernel_C::tg_decode_step,
 *                            torch_bindings.cpp:65-184, 227-264)
 *   mkd_reset_counters    <- extern "C" tg_launch_zero_regions(...),
 *                            taskgraph_kernel.cu:2000-2023 (bound as
 *                            tg_zero_regions, torch_bindings.cpp:186-225); here
 *                            it only runs at init or after a failed step, because
 *                            the step itself leaves every counter at zero
 *   mkd_launch_stages, mkd_graph_*  <- no kernel-level counterpart: the
 *                            reference's comparator arm is torch + CUDA Graph
 *                            (model_runner.py:378-416); here the comparator is a
 *                            captured hipGraph of this library's own per-op
 *                            kernels
 *   mkd_workspace_bytes   <- TaskGraphDecoder scratch sizing, taskgraph.py:213-249
 */
#ifndef MKD_ABI_H
#define MKD_ABI_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define MKD_ABI_VERSION 1

/* Compiled geometry: Qwen3-0.6B (reference model_spec.py:399-411). */
#define MKD_HIDDEN 1024
#define MKD_INTERMEDIATE 3072
#define MKD_NUM_LAYERS 28
#define MKD_NUM_Q_HEADS 16
#define MKD_NUM_KV_HEADS 8
#define MKD_HEAD_DIM 128
#define MKD_VOCAB 151936
#define MKD_MAX_POSITION 2048
#define MKD_MAX_BATCH 8
#define MKD_MAX_SPLITS 16
#define MKD_LAYER_PTRS 11
#define MKD_INST_WORDS 8
#define MKD_MAX_LM_SLOTS 1024

/* Per-layer weight pointer order (reference TgLayerWeightIdx, tg_abi.h:94-107). */
enum MkdLayerWeight {
  MKD_W_LN_IN = 0, MKD_W_Q = 1, MKD_W_K = 2, MKD_W_V = 3, MKD_W_Q_NORM = 4,
  MKD_W_K_NORM = 5, MKD_W_O = 6, MKD_W_LN_POST = 7, MKD_W_GATE = 8,
  MKD_W_UP = 9, MKD_W_DOWN = 10
};

/* Task opcodes of the instruction stream (reference TgOp, tg_abi.h:33-52). */
enum MkdOp {
  MKD_OP_NOP = 0,
  MKD_OP_QKV = 1,    /* residual add + input RMSNorm + rows of [Wq;Wk;Wv] */
  MKD_OP_ATTN = 2,   /* q/k norm + RoPE + KV write + one split of paged GQA attention */
  MKD_OP_OPROJ = 3,  /* rows of Wo */
  MKD_OP_GATEUP = 4, /* residual add + post-attn RMSNorm + gate/up row pairs + SiLU*mul */
  MKD_OP_DOWN = 5,   /* rows of Wd */
  MKD_OP_LMHEAD = 6  /* final RMSNorm + rows of the tied embedding + greedy argmax */
};

/* Instruction words (int32 x MKD_INST_WORDS). */
enum MkdInstWord {
  MKD_I_OP = 0, MKD_I_LAYER = 1, MKD_I_A0 = 2, MKD_I_A1 = 3, MKD_I_A2 = 4,
  MKD_I_WAIT = 5,      /* fan-in counter id to wait on, or -1 */
  MKD_I_WAIT_CNT = 6,  /* arrivals that counter reaches when the producers are done */
  MKD_I_SIGNAL = 7     /* fan-in counter id to arrive on after the task, or -1 */
};
/* Operand meaning: QKV/OPROJ/DOWN: A0 = first row, A1 = row count.
 * GATEUP: A0 = first intermediate channel, A1 = channel count.
 * ATTN: A0 = batch row * 8 + kv head, A1 = split index, A2 = split count.
 * LMHEAD: A0 = first vocab row, A1 = row count, A2 = argmax slot (0..slots-1),
 *         and WAIT_CNT of a LMHEAD word is unused; the slot count is
 *         MkdStepDesc.lm_slots. */

#define MKD_FLAG_ADVANCE 1u   /* after the step: input_ids[b] = token, cache_seqlens[b] += 1 */
#define MKD_FLAG_ZERO_FANIN 2u /* set by the persistent launch: last LM task clears fan-in counters */
#define MKD_FLAG_PK_V1 4u      /* persistent launch, first variant: no weight prefetch (A/B reference) */
#define MKD_FLAG_PK_V3 8u      /* reserved: a removed register-streaming variant (launches with it fail) */
#define MKD_FLAG_PK_TAGGED 16u /* persistent launch, tagged activation exchange (no counters) */

typedef struct MkdStepDesc {
  /* weights (device) */
  const uint64_t* layer_ptrs;   /* [num_layers][MKD_LAYER_PTRS] device pointers to bf16 tensors */
  const uint16_t* embed;        /* [vocab][hidden] bf16, also the tied LM head */
  const uint16_t* final_norm;   /* [hidden] bf16 */
  const float* rope_cos;        /* [MKD_MAX_POSITION][head_dim/2] fp32 */
  const float* rope_sin;
  /* paged KV cache: K and V views, each [layers][blocks][block_size][kv_heads][head_dim] bf16 */
  uint16_t* k_cache;
  uint16_t* v_cache;
  int64_t kv_layer_stride;      /* elements between consecutive layers of one view */
  int32_t num_blocks;
  int32_t block_size;
  const int32_t* page_table;    /* [rows][page_stride] physical block ids, padded with 0 */
  int32_t page_stride;
  int32_t _pad0;
  int32_t* cache_seqlens;       /* [rows] pre-decode KV length == this token's position */
  const int32_t* row_active;    /* [rows] 0 = skip the KV write (continuous batching) */
  int64_t* input_ids;           /* [rows] token ids of this step */
  /* outputs */
  int32_t* out_tokens;          /* [rows] greedy token ids */
  uint16_t* out_logits;         /* optional [rows][vocab] bf16 logits, NULL to skip */
  /* workspace from mkd_workspace_bytes(), zeroed by mkd_reset_counters() once */
  void* workspace;
  uint64_t workspace_bytes;
  /* step geometry */
  int32_t rows;                 /* live rows, 1..batch */
  int32_t batch;                /* compiled row bucket: 1, 2, 4 or 8 */
  int32_t num_layers;           /* 1..MKD_NUM_LAYERS (28 for the model) */
  int32_t lm_slots;             /* number of LMHEAD tasks (argmax partial slots) */
  uint32_t flags;               /* MKD_FLAG_* */
  int32_t _pad1;
  /* optional [grid][max_inst][4] uint64 timestamps (100 MHz device clock) of
   * the persistent kernel's tasks: start, dependency met, inputs staged, done;
   * NULL to skip (diagnostics only: written by the batch-8 kernel, and by every
   * batch's kernel in a library built with -DMKD_TRACE_TASKS) */
  uint64_t* trace;
} MkdStepDesc;

/* A task list uploaded to the device. For mkd_launch_persistent it is
 * [grid][max_inst][MKD_INST_WORDS] plus num_inst[grid]; for mkd_launch_stages
 * each stage is a contiguous run of instructions executed by one kernel. */
typedef struct MkdSchedule {
  const int32_t* inst;          /* device */
  const int32_t* num_inst;      /* device [grid] (persistent only) */
  int32_t grid;                 /* persistent: workgroups (<= CUs) */
  int32_t max_inst;             /* persistent: instructions per workgroup row */
} MkdSchedule;

typedef struct MkdStage {
  int32_t op;                   /* MkdOp of every instruction of the stage */
  int32_t layer;
  int32_t first;                /* index of the stage's first instruction in inst */
  int32_t count;                /* instructions (one workgroup each) */
} MkdStage;

int mkd_abi_version(void);
const char* mkd_last_error(void);
/* Compute units and LDS bytes per workgroup of device `device`. */
int mkd_device_info(int device, int32_t* num_cus, int32_t* lds_bytes);
/* Bytes of workspace a step needs (activations, attention partials, counters). */
uint64_t mkd_workspace_bytes(void);
/* Byte offset in the workspace of the 128-byte status line: the device error
 * word (uint32, 0 = ok) at +0; a decoder may point out_tokens at +64 so that one
 * 128-byte read returns the error word and the tokens together. */
uint64_t mkd_status_offset(void);
/* Zero every counter and the error word of the workspace (fill kernel, no memset node). */
int mkd_reset_counters(const MkdStepDesc* desc, void* stream);
/* One decode step as ONE persistent launch of `sched.grid` workgroups that walk
 * their instruction rows, waiting on / arriving at fan-in counters. */
int mkd_launch_persistent(const MkdStepDesc* desc, const MkdSchedule* sched, void* stream);
/* One decode step as one kernel launch per stage, same task bodies, no counters. */
int mkd_launch_stages(const MkdStepDesc* desc, const int32_t* inst,
                      const MkdStage* stages, int32_t num_stages, void* stream);
/* Read back the device error word (0 = ok); synchronizes `stream`. */
int mkd_check_error(const MkdStepDesc* desc, void* stream, int32_t* code);

/* Allocation-free variant of mkd_launch_persistent. No counterpart in the
 * reference: it is for callers that cannot allocate device memory (code under
 * hipGraph capture, tight serving loops, harnesses that forbid hipMalloc). The
 * descriptor's workspace/workspace_bytes are ignored; the step runs on a
 * library-owned scratch array of mkd_workspace_bytes() bytes per device (sized
 * for the maxima: batch 8, 28 layers, 16 attention splits, 1024 LM slots;
 * larger descriptors are rejected), looked up and cleared on the first call on
 * a device and held until the process ends. The caller passes inputs and
 * outputs as usual (out_tokens must be its own device memory) plus `status`, a
 * device int32 that receives the step's device error word (0 = ok); after an
 * error the scratch is cleared for the next call. No hipMalloc/hipFree or
 * allocating library call is made. All calls on one device share its scratch:
 * calls that overlap on one GPU (several streams or threads) race. */
int mkd_launch_persistent_noalloc(const MkdStepDesc* desc, const MkdSchedule* sched, int32_t* status,
                                  void* stream);

/* Captured hipGraph of a launch mode ("graph" comparator / replay path).
 * mode 0 = per-op stages of the generic task kernels (inst/stages/num_stages),
 * 1 = one persistent launch (sched), 2 = one persistent launch per schedule of
 * the array sched[0 .. num_stages-1] (the per-op comparator on the persistent
 * kernel's own task bodies: one stage per schedule, one task per workgroup).
 * `steps` consecutive decode steps are captured (use MKD_FLAG_ADVANCE to feed
 * each step's token to the next). */
int mkd_graph_create(const MkdStepDesc* desc, int32_t mode, const MkdSchedule* sched,
                     const int32_t* inst, const MkdStage* stages, int32_t num_stages,
                     int32_t steps, void* stream, void** graph_out);
int mkd_graph_launch(void* graph, void* stream);
int mkd_graph_destroy(void* graph);

#define MKD_OK 0
#define MKD_E_INVALID (-1)
#define MKD_E_HIP (-2)
#define MKD_E_DEVICE (-3)

#ifdef __cplusplus
}
#endif
#endif /* MKD_ABI_H */
