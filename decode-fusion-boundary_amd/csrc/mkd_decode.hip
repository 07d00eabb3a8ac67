// mkd_decode.hip -- kernels and C ABI of the MI355X Qwen3-0.6B decode step.
//
// Two launch modes run the same task bodies (mkd_tasks.h):
//  * persistent: one launch of <= #CU workgroups (one per CU); each walks its
//    row of the host-built instruction stream, spinning on fan-in counters
//    (sum of 8 sub-slots, relaxed agent-scope loads) before a task and
//    arriving on one afterwards. The last LM-head task clears the fan-in
//    counters, so a step leaves the workspace ready for the next without a
//    zeroing pass.
//  * stages: one kernel per stage of the same instruction list; kernel
//    boundaries order the stages; captured into a hipGraph by mkd_graph_create.
#include <hip/hip_runtime.h>

#include <cstdio>
#include <cstring>
#include <mutex>
#include <string>
#include <vector>

#include "mkd_pk4.h"

using namespace mkd;

namespace {

thread_local std::string g_last_error;

int fail(int code, const std::string& msg) {
  g_last_error = msg;
  return code;
}

int hip_fail(hipError_t e, const char* what) {
  return fail(MKD_E_HIP, std::string(what) + ": " + hipGetErrorString(e));
}

#define MKD_HIP(call)                                    \
  do {                                                   \
    hipError_t e_ = (call);                              \
    if (e_ != hipSuccess) return hip_fail(e_, #call);    \
  } while (0)

// Spin timeout for a fan-in wait: ~4 s of the 100 MHz constant clock. A wait
// that expires records ERR_TIMEOUT and the workgroup leaves the kernel, so a
// broken schedule ends the launch instead of hanging the device.
constexpr uint64_t WAIT_TICKS = 400000000ull;

__device__ bool wait_fanin(const Ws& ws, int fanin, uint32_t target, int* sh_abort) {
  const int lane = threadIdx.x;
  if (threadIdx.x < 64) {
    const uint64_t t_start = wall_clock64();
    bool ok = false;
    while (true) {
      uint32_t v = lane < FANIN_SUBSLOTS ? ld_co(ws.line(CTR_FANIN_BASE + fanin * FANIN_SUBSLOTS + lane)) : 0u;
#pragma unroll
      for (int o = 1; o < FANIN_SUBSLOTS; o <<= 1) v += __shfl_xor(v, o, 64);
      v = __shfl(v, 0, 64);
      if (v >= target) { ok = true; break; }
      if (ld_co(ws.line(CTR_ERR)) != 0u) break;
      if (wall_clock64() - t_start > WAIT_TICKS) {
        if (lane == 0) st_co(ws.line(CTR_ERR), ERR_TIMEOUT);
        break;
      }
      __builtin_amdgcn_s_sleep(1);
    }
    if (lane == 0) *sh_abort = ok ? 0 : 1;
  }
  __syncthreads();
  return *sh_abort == 0;
}

template <int B>
__device__ bool run_task(const MkdStepDesc& d, const Ws& ws, const int32_t* w, uint8_t* smem) {
  const int op = w[MKD_I_OP], layer = w[MKD_I_LAYER];
  const int a0 = w[MKD_I_A0], a1 = w[MKD_I_A1], a2 = w[MKD_I_A2];
  switch (op) {
    case MKD_OP_QKV: task_qkv<B>(d, ws, layer, a0, a1, smem); return true;
    case MKD_OP_ATTN: return task_attn<B>(d, ws, layer, a0, a1, a2, smem);
    case MKD_OP_OPROJ:
      task_proj<B, QS>(wptr(d, layer, MKD_W_O), ws.attn(), ws.hid_a(), a0, a1, smem);
      return true;
    case MKD_OP_GATEUP: task_gateup<B>(d, ws, layer, a0, a1, smem); return true;
    case MKD_OP_DOWN:
      task_proj<B, I>(wptr(d, layer, MKD_W_DOWN), ws.act(), ws.hid_f(), a0, a1, smem);
      return true;
    case MKD_OP_LMHEAD: task_lmhead<B>(d, ws, a0, a1, a2, smem); return false;
    default: return false;
  }
}

template <int B>
__global__ __launch_bounds__(NT, 1) void k_persistent(MkdStepDesc d, MkdSchedule s) {
  __shared__ __attribute__((aligned(16))) uint8_t smem[SMEM_BYTES];
  __shared__ int sh_abort;
  const Ws ws{reinterpret_cast<uint8_t*>(d.workspace)};
  const int n = s.num_inst[blockIdx.x];
  const int32_t* row = s.inst + (size_t)blockIdx.x * s.max_inst * MKD_INST_WORDS;
  for (int i = 0; i < n; i++) {
    const int32_t* w = row + i * MKD_INST_WORDS;
    __syncthreads();  // the previous task is done with smem
    const int wait = w[MKD_I_WAIT];
    if (wait >= 0 && !wait_fanin(ws, wait, (uint32_t)w[MKD_I_WAIT_CNT], &sh_abort)) return;
    const bool produced = run_task<B>(d, ws, w, smem);
    const int signal = w[MKD_I_SIGNAL];
    if (signal >= 0 && produced) {
      drain();
      __syncthreads();
      if (threadIdx.x == 0)
        add_co(ws.line(CTR_FANIN_BASE + signal * FANIN_SUBSLOTS + (blockIdx.x & (FANIN_SUBSLOTS - 1))), 1u);
    }
  }
}

template <int B, int OP>
__global__ __launch_bounds__(NT) void k_stage(MkdStepDesc d, const int32_t* inst) {
  __shared__ __attribute__((aligned(16))) uint8_t smem[SMEM_BYTES];
  const Ws ws{reinterpret_cast<uint8_t*>(d.workspace)};
  const int32_t* w = inst + (size_t)blockIdx.x * MKD_INST_WORDS;
  if (w[MKD_I_OP] != OP) {
    if (threadIdx.x == 0) st_co(ws.line(CTR_ERR), ERR_BAD_INST);
    return;
  }
  run_task<B>(d, ws, w, smem);
}

__global__ void k_reset(uint32_t* ctr, int n_u32) {
  for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < n_u32; i += gridDim.x * blockDim.x) ctr[i] = 0u;
}

int validate(const MkdStepDesc* d) {
  if (d == nullptr) return fail(MKD_E_INVALID, "null step descriptor");
  if (d->batch != 1 && d->batch != 2 && d->batch != 4 && d->batch != 8)
    return fail(MKD_E_INVALID, "batch must be 1, 2, 4 or 8; got " + std::to_string(d->batch));
  if (d->rows < 1 || d->rows > d->batch)
    return fail(MKD_E_INVALID, "rows must be in [1, batch]; got " + std::to_string(d->rows));
  if (d->num_layers < 1 || d->num_layers > MKD_NUM_LAYERS)
    return fail(MKD_E_INVALID, "num_layers must be in [1, 28]");
  if (d->lm_slots < 1 || d->lm_slots > MKD_MAX_LM_SLOTS)
    return fail(MKD_E_INVALID, "lm_slots must be in [1, 1024]");
  if (d->workspace == nullptr || d->workspace_bytes < WORKSPACE_BYTES)
    return fail(MKD_E_INVALID, "workspace missing or smaller than mkd_workspace_bytes()");
  if (d->block_size < 1 || d->num_blocks < 1 || d->page_stride < 1)
    return fail(MKD_E_INVALID, "invalid paged-KV geometry");
  if ((MKD_MAX_POSITION + d->block_size - 1) / d->block_size > MAX_PAGES)
    return fail(MKD_E_INVALID, "block_size too small: a 2048-token context needs more than 64 blocks");
  const void* ptrs[] = {d->layer_ptrs, d->embed, d->final_norm, d->rope_cos, d->rope_sin, d->k_cache,
                        d->v_cache, d->page_table, d->cache_seqlens, d->row_active, d->input_ids, d->out_tokens};
  for (const void* p : ptrs)
    if (p == nullptr) return fail(MKD_E_INVALID, "null device pointer in step descriptor");
  return MKD_OK;
}

// Per-device launch state of one persistent kernel: the dynamic-LDS attribute
// is set and the co-residency bound measured on the first launch on a device.
constexpr int MAX_DEVICES = 64;
struct PkState {
  bool ready = false;
  int blocks_per_cu = 0;
};
std::mutex g_pk_mu;

// Make `kern` launchable on the current device with `lds` bytes of dynamic LDS
// and check that a grid of `grid` workgroups of `threads` can all be resident
// at once (the persistent kernels' workgroups wait on each other, so a
// workgroup that could not start would leave the others spinning until their
// bounded waits give up).
int pk_ready(PkState (&state)[MAX_DEVICES], const void* kern, int threads, int lds, int grid) {
  int dev = 0, cus = 0;
  MKD_HIP(hipGetDevice(&dev));
  if (dev < 0 || dev >= MAX_DEVICES) return fail(MKD_E_INVALID, "device index out of range");
  std::lock_guard<std::mutex> lock(g_pk_mu);
  PkState& st = state[dev];
  if (!st.ready) {
    if (lds > 0) MKD_HIP(hipFuncSetAttribute(kern, hipFuncAttributeMaxDynamicSharedMemorySize, lds));
    int nb = 0;
    MKD_HIP(hipOccupancyMaxActiveBlocksPerMultiprocessor(&nb, kern, threads, (size_t)lds));
    st.blocks_per_cu = nb;
    st.ready = true;
  }
  MKD_HIP(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev));
  if (st.blocks_per_cu < 1 || grid > cus * st.blocks_per_cu)
    return fail(MKD_E_INVALID, "persistent grid of " + std::to_string(grid) + " workgroups cannot be co-resident: " +
                                   std::to_string(cus) + " compute units x " + std::to_string(st.blocks_per_cu) +
                                   " resident workgroups each");
  return MKD_OK;
}

template <int B>
int launch_persistent_b(const MkdStepDesc& d, const MkdSchedule& s, hipStream_t st) {
  static PkState st_v1[MAX_DEVICES], st_tagged[MAX_DEVICES], st_dma[MAX_DEVICES];  // per instantiation
  int rc = MKD_OK;
  if (d.flags & MKD_FLAG_PK_V1) {
    rc = pk_ready(st_v1, reinterpret_cast<const void*>(k_persistent<B>), NT, 0, s.grid);
    if (rc) return rc;
    hipLaunchKernelGGL(k_persistent<B>, dim3(s.grid), dim3(NT), 0, st, d, s);
  } else if (d.flags & MKD_FLAG_PK_TAGGED) {
    // its DMA waves stage 32-position KV chunks that must not straddle a cache block
    if (d.block_size % KV_CHUNK != 0)
      return fail(MKD_E_INVALID, "the tagged persistent kernel needs a block_size that is a multiple of 32");
    rc = pk_ready(st_tagged, reinterpret_cast<const void*>(k_persistent4<B>), PK_THREADS, PkCfg<B>::LDS_BYTES, s.grid);
    if (rc) return rc;
    hipLaunchKernelGGL(k_persistent4<B>, dim3(s.grid), dim3(PK_THREADS), PkCfg<B>::LDS_BYTES, st, d, s);
  } else if (d.flags & MKD_FLAG_PK_V3) {
    return fail(MKD_E_INVALID, "the register-streaming persistent variant was removed");
  } else {
    rc = pk_ready(st_dma, reinterpret_cast<const void*>(k_persistent2<B>), PK_THREADS, PkCfg<B>::LDS_BYTES, s.grid);
    if (rc) return rc;
    hipLaunchKernelGGL(k_persistent2<B>, dim3(s.grid), dim3(PK_THREADS), PkCfg<B>::LDS_BYTES, st, d, s);
  }
  MKD_HIP(hipGetLastError());
  return MKD_OK;
}

template <int B>
int launch_stage_b(const MkdStepDesc& d, const int32_t* inst, const MkdStage& sg, hipStream_t st) {
  const int32_t* first = inst + (size_t)sg.first * MKD_INST_WORDS;
  const dim3 grid(sg.count), block(NT);
  switch (sg.op) {
    case MKD_OP_QKV: hipLaunchKernelGGL((k_stage<B, MKD_OP_QKV>), grid, block, 0, st, d, first); break;
    case MKD_OP_ATTN: hipLaunchKernelGGL((k_stage<B, MKD_OP_ATTN>), grid, block, 0, st, d, first); break;
    case MKD_OP_OPROJ: hipLaunchKernelGGL((k_stage<B, MKD_OP_OPROJ>), grid, block, 0, st, d, first); break;
    case MKD_OP_GATEUP: hipLaunchKernelGGL((k_stage<B, MKD_OP_GATEUP>), grid, block, 0, st, d, first); break;
    case MKD_OP_DOWN: hipLaunchKernelGGL((k_stage<B, MKD_OP_DOWN>), grid, block, 0, st, d, first); break;
    case MKD_OP_LMHEAD: hipLaunchKernelGGL((k_stage<B, MKD_OP_LMHEAD>), grid, block, 0, st, d, first); break;
    default: return fail(MKD_E_INVALID, "unknown stage op " + std::to_string(sg.op));
  }
  MKD_HIP(hipGetLastError());
  return MKD_OK;
}

int do_persistent(const MkdStepDesc* d, const MkdSchedule* s, hipStream_t st) {
  int rc = validate(d);
  if (rc) return rc;
  if (s == nullptr || s->inst == nullptr || s->num_inst == nullptr || s->grid < 1 || s->max_inst < 1)
    return fail(MKD_E_INVALID, "invalid persistent schedule");
  MkdStepDesc dd = *d;
  dd.flags |= MKD_FLAG_ZERO_FANIN;
  switch (d->batch) {
    case 1: return launch_persistent_b<1>(dd, *s, st);
    case 2: return launch_persistent_b<2>(dd, *s, st);
    case 4: return launch_persistent_b<4>(dd, *s, st);
    default: return launch_persistent_b<8>(dd, *s, st);
  }
}

int do_stages(const MkdStepDesc* d, const int32_t* inst, const MkdStage* stages, int32_t n, hipStream_t st) {
  int rc = validate(d);
  if (rc) return rc;
  if (inst == nullptr || stages == nullptr || n < 1) return fail(MKD_E_INVALID, "empty stage list");
  MkdStepDesc dd = *d;
  dd.flags &= ~MKD_FLAG_ZERO_FANIN;
  for (int i = 0; i < n; i++) {
    if (stages[i].count < 1) return fail(MKD_E_INVALID, "stage with no tasks");
    switch (d->batch) {
      case 1: rc = launch_stage_b<1>(dd, inst, stages[i], st); break;
      case 2: rc = launch_stage_b<2>(dd, inst, stages[i], st); break;
      case 4: rc = launch_stage_b<4>(dd, inst, stages[i], st); break;
      default: rc = launch_stage_b<8>(dd, inst, stages[i], st); break;
    }
    if (rc) return rc;
  }
  return MKD_OK;
}

struct GraphHandle {
  hipGraph_t graph = nullptr;
  hipGraphExec_t exec = nullptr;
};

// After a step of the allocation-free entry point: copy the device error word
// to the caller's status int and, when it is set, clear the counters and the
// tagged exchange (error word last), so the next call starts clean. One
// workgroup: every thread has read the error word before any clears it.
__global__ __launch_bounds__(1024) void k_status_finish(uint8_t* ws, int32_t* status) {
  uint32_t* ctr = reinterpret_cast<uint32_t*>(ws + OFF_CTR);
  const uint32_t err = ld_co(ctr);
  __syncthreads();
  if (threadIdx.x == 0) *status = (int32_t)err;
  if (err == 0u) return;
  const int n = (int)((WORKSPACE_BYTES - OFF_CTR) / 4);
  for (int i = 1 + threadIdx.x; i < n; i += blockDim.x) ctr[i] = 0u;
  __syncthreads();
  if (threadIdx.x == 0) st_co(ctr, 0u);
}

}  // namespace

// Workspace of the allocation-free entry point (mkd_launch_persistent_noalloc):
// one copy per device, WORKSPACE_BYTES (sized for the library's maxima: batch
// 8, 28 layers, 16 attention splits, 1024 LM slots), held until the process
// ends. Host code uses only the per-device address from hipGetSymbolAddress,
// never this name.
static __device__ __align__(256) uint8_t scratch[WORKSPACE_BYTES];

namespace {

std::mutex g_scratch_mu;
void* g_scratch_ptr[MAX_DEVICES] = {};

// Address of this device's scratch, looked up (and cleared on `st`) on the
// first call on the device.
int scratch_for_device(hipStream_t st, void** out) {
  int dev = 0;
  MKD_HIP(hipGetDevice(&dev));
  if (dev < 0 || dev >= MAX_DEVICES) return fail(MKD_E_INVALID, "device index out of range");
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_ptr[dev] == nullptr) {
    void* ptr = nullptr;
    MKD_HIP(hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)));
    if (ptr == nullptr) return fail(MKD_E_HIP, "hipGetSymbolAddress returned a null scratch address");
    uint32_t* ctr = reinterpret_cast<uint32_t*>(reinterpret_cast<uint8_t*>(ptr) + OFF_CTR);
    hipLaunchKernelGGL(k_reset, dim3(256), dim3(256), 0, st, ctr, (int)((WORKSPACE_BYTES - OFF_CTR) / 4));
    MKD_HIP(hipGetLastError());
    g_scratch_ptr[dev] = ptr;
  }
  *out = g_scratch_ptr[dev];
  return MKD_OK;
}

}  // namespace

extern "C" {

int mkd_abi_version(void) { return MKD_ABI_VERSION; }

const char* mkd_last_error(void) { return g_last_error.c_str(); }

int mkd_device_info(int device, int32_t* num_cus, int32_t* lds_bytes) {
  int v = 0;
  MKD_HIP(hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, device));
  if (num_cus) *num_cus = v;
  MKD_HIP(hipDeviceGetAttribute(&v, hipDeviceAttributeMaxSharedMemoryPerBlock, device));
  if (lds_bytes) *lds_bytes = v;
  return MKD_OK;
}

uint64_t mkd_workspace_bytes(void) { return WORKSPACE_BYTES; }

uint64_t mkd_status_offset(void) { return OFF_CTR; }

int mkd_reset_counters(const MkdStepDesc* d, void* stream) {
  if (d == nullptr || d->workspace == nullptr || d->workspace_bytes < WORKSPACE_BYTES)
    return fail(MKD_E_INVALID, "workspace missing or too small");
  // counters, the epoch and every tagged word: no stale tag can match after a reset
  uint32_t* ctr = reinterpret_cast<uint32_t*>(reinterpret_cast<uint8_t*>(d->workspace) + OFF_CTR);
  const int n = (int)((WORKSPACE_BYTES - OFF_CTR) / 4);
  hipLaunchKernelGGL(k_reset, dim3(256), dim3(256), 0, (hipStream_t)stream, ctr, n);
  MKD_HIP(hipGetLastError());
  return MKD_OK;
}

int mkd_launch_persistent(const MkdStepDesc* d, const MkdSchedule* s, void* stream) {
  return do_persistent(d, s, (hipStream_t)stream);
}

int mkd_launch_persistent_noalloc(const MkdStepDesc* d, const MkdSchedule* s, int32_t* status, void* stream) {
  if (d == nullptr) return fail(MKD_E_INVALID, "null step descriptor");
  if (status == nullptr) return fail(MKD_E_INVALID, "null status pointer");
  hipStream_t st = (hipStream_t)stream;
  void* ws = nullptr;
  int rc = scratch_for_device(st, &ws);
  if (rc) return rc;
  MkdStepDesc dd = *d;
  dd.workspace = ws;
  dd.workspace_bytes = WORKSPACE_BYTES;
  const uint8_t* out_lo = reinterpret_cast<const uint8_t*>(d->out_tokens);
  const uint8_t* ws_lo = reinterpret_cast<const uint8_t*>(ws);
  if (out_lo >= ws_lo && out_lo < ws_lo + WORKSPACE_BYTES)
    return fail(MKD_E_INVALID, "out_tokens must not point into the library's scratch");
  rc = do_persistent(&dd, s, st);  // validates rows/batch/layers/slots against the scratch's maxima
  if (rc) return rc;
  hipLaunchKernelGGL(k_status_finish, dim3(1), dim3(1024), 0, st, reinterpret_cast<uint8_t*>(ws), status);
  MKD_HIP(hipGetLastError());
  return MKD_OK;
}

int mkd_launch_stages(const MkdStepDesc* d, const int32_t* inst, const MkdStage* stages, int32_t n, void* stream) {
  return do_stages(d, inst, stages, n, (hipStream_t)stream);
}

int mkd_check_error(const MkdStepDesc* d, void* stream, int32_t* code) {
  if (d == nullptr || d->workspace == nullptr) return fail(MKD_E_INVALID, "workspace missing");
  uint32_t host = 0;
  const uint8_t* src = reinterpret_cast<const uint8_t*>(d->workspace) + OFF_CTR;
  MKD_HIP(hipMemcpyAsync(&host, src, 4, hipMemcpyDeviceToHost, (hipStream_t)stream));
  MKD_HIP(hipStreamSynchronize((hipStream_t)stream));
  if (code) *code = (int32_t)host;
  if (host == ERR_TIMEOUT) return fail(MKD_E_DEVICE, "a persistent-kernel dependency wait timed out");
  if (host == ERR_BAD_INST) return fail(MKD_E_DEVICE, "a stage kernel met an instruction of another op");
  if (host != 0) return fail(MKD_E_DEVICE, "device error word " + std::to_string(host));
  return MKD_OK;
}

int mkd_graph_create(const MkdStepDesc* d, int32_t mode, const MkdSchedule* s, const int32_t* inst,
                     const MkdStage* stages, int32_t num_stages, int32_t steps, void* stream, void** out) {
  if (out == nullptr) return fail(MKD_E_INVALID, "null graph handle");
  if (steps < 1) return fail(MKD_E_INVALID, "steps must be >= 1");
  if (mode < 0 || mode > 2) return fail(MKD_E_INVALID, "graph mode must be 0, 1 or 2");
  if (mode == 2 && (s == nullptr || num_stages < 1))
    return fail(MKD_E_INVALID, "mode 2 needs an array of num_stages >= 1 persistent schedules");
  int rc = validate(d);
  if (rc) return rc;
  hipStream_t cap = nullptr;
  MKD_HIP(hipStreamCreateWithFlags(&cap, hipStreamNonBlocking));
  auto* g = new GraphHandle();
  hipError_t e = hipStreamBeginCapture(cap, hipStreamCaptureModeThreadLocal);
  if (e != hipSuccess) {
    delete g;
    hipStreamDestroy(cap);
    return hip_fail(e, "hipStreamBeginCapture");
  }
  for (int i = 0; i < steps && rc == MKD_OK; i++) {
    if (mode == 2) {
      // one persistent launch per schedule of the array, in order
      for (int k = 0; k < num_stages && rc == MKD_OK; k++) rc = do_persistent(d, s + k, cap);
    } else {
      rc = mode == 1 ? do_persistent(d, s, cap) : do_stages(d, inst, stages, num_stages, cap);
    }
  }
  e = hipStreamEndCapture(cap, &g->graph);
  if (rc == MKD_OK && e != hipSuccess) rc = hip_fail(e, "hipStreamEndCapture");
  if (rc == MKD_OK) {
    e = hipGraphInstantiate(&g->exec, g->graph, nullptr, nullptr, 0);
    if (e != hipSuccess) rc = hip_fail(e, "hipGraphInstantiate");
  }
  hipStreamDestroy(cap);
  if (rc != MKD_OK) {
    if (g->exec) hipGraphExecDestroy(g->exec);
    if (g->graph) hipGraphDestroy(g->graph);
    delete g;
    return rc;
  }
  (void)stream;
  *out = g;
  return MKD_OK;
}

int mkd_graph_launch(void* graph, void* stream) {
  if (graph == nullptr) return fail(MKD_E_INVALID, "null graph");
  MKD_HIP(hipGraphLaunch(static_cast<GraphHandle*>(graph)->exec, (hipStream_t)stream));
  return MKD_OK;
}

int mkd_graph_destroy(void* graph) {
  if (graph == nullptr) return MKD_OK;
  auto* g = static_cast<GraphHandle*>(graph);
  if (g->exec) hipGraphExecDestroy(g->exec);
  if (g->graph) hipGraphDestroy(g->graph);
  delete g;
  return MKD_OK;
}

}  // extern "C"
