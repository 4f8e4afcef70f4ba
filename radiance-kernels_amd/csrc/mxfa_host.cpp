// libmxfa.so: C ABI over the gfx950 code object mxfa_kernels.hsaco.
//
// Replaces the reference's launch path (mu_schedule(fa_entry, nullptr, occupancy),
// lib/src/mu_schedule.cpp:83-104, started from main() in
// kernels/flash_attention_mx_gqa/kernel.cpp:186-191) with hipModuleLaunchKernel on
// the caller's stream.  One hipModule per device is loaded lazily (or by
// mxfa_init) and kept until mxfa_shutdown.  Host code only: built with g++ against
// libamdhip64; the kernels are compiled separately by hipcc --genco.
#include "mxfa.h"

#include <dlfcn.h>
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <mutex>
#include <string>
#include <unordered_map>

#include "mxfa_args.h"

namespace {

thread_local std::string g_err;

mxfa_status fail(mxfa_status st, const std::string& msg) {
  g_err = msg;
  return st;
}

#define MXFA_HIP(call)                                                                         \
  do {                                                                                         \
    hipError_t e_ = (call);                                                                    \
    if (e_ != hipSuccess) return fail(MXFA_ERR_HIP, std::string(#call) + ": " + hipGetErrorString(e_)); \
  } while (0)

const char* const kKernelNames[] = {
    "mxfa_quant_rows_e4m3",    "mxfa_quant_rows_e3m2",    "mxfa_quant_cols_e4m3", "mxfa_quant_cols_e3m2",
    "mxfa_softmax_requant_rows",     "mxfa_fill_normal_f32",
    "mxfa_decode_d64",         "mxfa_decode_d128",        "mxfa_decode_d256",     "mxfa_decode_d64_softcap",
    "mxfa_decode_d128_softcap", "mxfa_decode_d256_softcap", "mxfa_decode_combine", "mxfa_kv_append_e4m3",
    "mxfa_kv_append_e3m2",     "mxfa_kv_tail_update",     "mxfa_quant_rows_r4",
    "mxfa_decode_d64_r2", "mxfa_decode_d128_r2",
    "mxfa_decode_d256_r2",     "mxfa_decode_d64_softcap_r2", "mxfa_decode_d128_softcap_r2",
    "mxfa_decode_d256_softcap_r2", "mxfa_gemm", "mxfa_gemm_ae3m2", "mxfa_gemm_be3m2", "mxfa_gemm_ae3m2_be3m2",
    "mxfa_k_to_bf16",          "mxfa_prefill3_d64",       "mxfa_prefill3_d128",   "mxfa_prefill3_d64_softcap",
    "mxfa_prefill3_d128_softcap", "mxfa_prefill3_d64_r2", "mxfa_prefill3_d128_r2", "mxfa_prefill3_d64_softcap_r2",
    "mxfa_prefill3_d128_softcap_r2",
    "mxfa_prefill3_d256",      "mxfa_prefill3_d256_softcap", "mxfa_prefill3_d256_r2", "mxfa_prefill3_d256_softcap_r2",
    "mxfa_prefill3_trace_d64", "mxfa_prefill3_trace_d128", "mxfa_prefill3_trace_d256",
    "mxfa_prefill3_trace_d64_softcap", "mxfa_prefill3_trace_d128_softcap", "mxfa_prefill3_trace_d256_softcap",
    "mxfa_prefill3_trace_d64_r2", "mxfa_prefill3_trace_d128_r2", "mxfa_prefill3_trace_d256_r2",
    "mxfa_prefill3_trace_d64_softcap_r2", "mxfa_prefill3_trace_d128_softcap_r2", "mxfa_prefill3_trace_d256_softcap_r2",
    "mxfa_gemm_dma", "mxfa_gemm_skinny_t1", "mxfa_gemm_skinny_t2", "mxfa_gemm_skinny_t4",
    "mxfa_prefill3n_d64", "mxfa_prefill3n_d128", "mxfa_prefill3n_d256", "mxfa_prefill3n_d64_softcap",
    "mxfa_prefill3n_d128_softcap", "mxfa_prefill3n_d256_softcap", "mxfa_prefill3n_d64_r2", "mxfa_prefill3n_d128_r2",
    "mxfa_prefill3n_d256_r2", "mxfa_prefill3n_d64_softcap_r2", "mxfa_prefill3n_d128_softcap_r2",
    "mxfa_prefill3n_d256_softcap_r2",
    "mxfa_prefill3n_d64_e3m2", "mxfa_prefill3n_d128_e3m2", "mxfa_prefill3n_d256_e3m2",
    "mxfa_prefill3n_d64_softcap_e3m2", "mxfa_prefill3n_d128_softcap_e3m2", "mxfa_prefill3n_d256_softcap_e3m2",
    "mxfa_prefill3n_d64_r2_e3m2", "mxfa_prefill3n_d128_r2_e3m2", "mxfa_prefill3n_d256_r2_e3m2",
    "mxfa_prefill3n_d64_softcap_r2_e3m2", "mxfa_prefill3n_d128_softcap_r2_e3m2", "mxfa_prefill3n_d256_softcap_r2_e3m2",
    "mxfa_quant_cols_e3m2_blk", "mxfa_kv_append_e3m2_blk",
#define MXFA_BLK_NAMES(D)                                                                                      \
  "mxfa_prefill3_d" #D "_blk", "mxfa_prefill3_d" #D "_softcap_blk", "mxfa_prefill3_d" #D "_r2_blk",            \
      "mxfa_prefill3_d" #D "_softcap_r2_blk", "mxfa_prefill3n_d" #D "_blk", "mxfa_prefill3n_d" #D "_softcap_blk", \
      "mxfa_prefill3n_d" #D "_r2_blk", "mxfa_prefill3n_d" #D "_softcap_r2_blk"
    MXFA_BLK_NAMES(64), MXFA_BLK_NAMES(128), MXFA_BLK_NAMES(256),
#define MXFA_DECODE_BLK_NAMES(D)                                                            \
  "mxfa_decode_d" #D "_blk", "mxfa_decode_d" #D "_softcap_blk", "mxfa_decode_d" #D "_r2_blk", \
      "mxfa_decode_d" #D "_softcap_r2_blk"
    MXFA_DECODE_BLK_NAMES(64), MXFA_DECODE_BLK_NAMES(128), MXFA_DECODE_BLK_NAMES(256),
};
constexpr int kNumKernels = sizeof(kKernelNames) / sizeof(kKernelNames[0]);

struct DeviceModule {
  hipModule_t mod = nullptr;
  hipFunction_t fn[kNumKernels] = {};
  void* decode_scratch = nullptr;     // this device's address of mxfa_decode_scratch
  size_t decode_scratch_bytes = 0;
};

std::mutex g_mu;
std::unordered_map<int, DeviceModule> g_mods;

std::string code_object_path() {
  if (const char* env = getenv("MXFA_HSACO")) return env;
  Dl_info info;
  if (dladdr(reinterpret_cast<void*>(&mxfa_version), &info) && info.dli_fname) {
    std::string p(info.dli_fname);
    size_t slash = p.rfind('/');
    return (slash == std::string::npos ? std::string(".") : p.substr(0, slash)) + "/mxfa_kernels.hsaco";
  }
  return "mxfa_kernels.hsaco";
}

// Module of the current device (loaded on first use).
mxfa_status module_for_current(DeviceModule** out) {
  int dev = -1;
  MXFA_HIP(hipGetDevice(&dev));
  std::lock_guard<std::mutex> lk(g_mu);
  auto it = g_mods.find(dev);
  if (it != g_mods.end()) {
    *out = &it->second;
    return MXFA_OK;
  }
  hipDeviceProp_t prop;
  MXFA_HIP(hipGetDeviceProperties(&prop, dev));
  if (std::strncmp(prop.gcnArchName, "gfx950", 6) != 0)
    return fail(MXFA_ERR_UNSUPPORTED, std::string("device ") + std::to_string(dev) + " is " + prop.gcnArchName +
                                          "; libmxfa is built for gfx950 (MI355X) only");
  DeviceModule dm;
  std::string path = code_object_path();
  hipError_t e = hipModuleLoad(&dm.mod, path.c_str());
  if (e != hipSuccess) return fail(MXFA_ERR_MODULE, "hipModuleLoad(" + path + "): " + hipGetErrorString(e));
  for (int i = 0; i < kNumKernels; i++) {
    e = hipModuleGetFunction(&dm.fn[i], dm.mod, kKernelNames[i]);
    if (e != hipSuccess) {
      (void)hipModuleUnload(dm.mod);
      return fail(MXFA_ERR_MODULE, std::string("kernel ") + kKernelNames[i] + " missing from " + path);
    }
  }
  // The device address of the decode scratch array in this device's copy of the module (the
  // module-API form of hipGetSymbolAddress): taken here, with the device current, and only
  // this address is ever passed to a kernel.
  hipDeviceptr_t sp = nullptr;
  e = hipModuleGetGlobal(&sp, &dm.decode_scratch_bytes, dm.mod, "mxfa_decode_scratch");
  if (e != hipSuccess || !sp || dm.decode_scratch_bytes < MXFA_DECODE_SCRATCH_BYTES) {
    (void)hipModuleUnload(dm.mod);
    return fail(MXFA_ERR_MODULE, std::string("hipModuleGetGlobal(mxfa_decode_scratch) in ") + path + ": " +
                                     (e != hipSuccess ? hipGetErrorString(e) : "missing or too small"));
  }
  dm.decode_scratch = reinterpret_cast<void*>(sp);
  auto res = g_mods.emplace(dev, dm);
  *out = &res.first->second;
  return MXFA_OK;
}

// Module of the current device if it is already loaded (never loads: no allocation).
mxfa_status loaded_module_for_current(DeviceModule** out) {
  int dev = -1;
  MXFA_HIP(hipGetDevice(&dev));
  std::lock_guard<std::mutex> lk(g_mu);
  auto it = g_mods.find(dev);
  if (it == g_mods.end())
    return fail(MXFA_ERR_MODULE, "no code object loaded on device " + std::to_string(dev) +
                                     ": call mxfa_init() on it before mxfa_decode_noalloc");
  *out = &it->second;
  return MXFA_OK;
}

hipFunction_t fn_by_name(DeviceModule* dm, const char* name) {
  for (int i = 0; i < kNumKernels; i++)
    if (std::strcmp(kKernelNames[i], name) == 0) return dm->fn[i];
  return nullptr;
}

// MXFA_PREFILL_LDS_PAD=<bytes>: that much dynamic LDS added to every prefill launch, which
// lowers how many workgroups share a CU without changing the code object (an occupancy
// measurement; unset, the launches use their static LDS only)
unsigned prefill_lds_pad(const char* name) {
  if (std::strncmp(name, "mxfa_prefill3", 13) != 0) return 0;
  const char* env = getenv("MXFA_PREFILL_LDS_PAD");
  const long v = env ? atol(env) : 0;
  return v > 0 && v <= 96 * 1024 ? (unsigned)v : 0;
}

mxfa_status launch(DeviceModule* dm, const char* name, dim3 grid, dim3 block, void** args, void* stream) {
  hipFunction_t f = fn_by_name(dm, name);
  if (!f) return fail(MXFA_ERR_MODULE, std::string("unknown kernel ") + name);
  MXFA_HIP(hipModuleLaunchKernel(f, grid.x, grid.y, grid.z, block.x, block.y, block.z, prefill_lds_pad(name),
                                 reinterpret_cast<hipStream_t>(stream), args, nullptr));
  return MXFA_OK;
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// A launch's x extent in work-items (grid.x * block.x) is a 32-bit count in the dispatch
// packet: a call that would need more is refused before any device work.
mxfa_status check_grid(int64_t blocks, int threads) {
  if (blocks * threads > (int64_t)UINT32_MAX)
    return fail(MXFA_ERR_UNSUPPORTED, "the call needs more than 2^32 work-items in one launch: split it");
  return MXFA_OK;
}

mxfa_status check_params(const mxfa_attn_params* p, bool decode) {
  if (!p) return fail(MXFA_ERR_INVALID_ARG, "params is NULL");
  if (p->batch < 1 || p->num_q_heads < 1 || p->num_kv_heads < 1 || p->seq_q < 1 || p->seq_k < 1)
    return fail(MXFA_ERR_INVALID_ARG, "batch, heads, seq_q and seq_k must be >= 1");
  if (p->num_q_heads % p->num_kv_heads)
    return fail(MXFA_ERR_INVALID_ARG, "num_q_heads must be a multiple of num_kv_heads");
  if (p->head_dim % 32) return fail(MXFA_ERR_INVALID_ARG, "head_dim must be a multiple of 32");
  if (p->head_dim != 64 && p->head_dim != 128 && p->head_dim != 256)
    return fail(MXFA_ERR_UNSUPPORTED, "head_dim must be 64, 128 or 256");
  if (p->seq_k % 32) return fail(MXFA_ERR_INVALID_ARG, "seq_k must be a multiple of 32 (V scale blocks)");
  if (p->q_pos0 < 0 || p->window < 0) return fail(MXFA_ERR_INVALID_ARG, "q_pos0 and window must be >= 0");
  if (!(p->softmax_scale > 0.0f) || !std::isfinite(p->softmax_scale))
    return fail(MXFA_ERR_INVALID_ARG, "softmax_scale must be finite and > 0");
  if (!(p->softcap >= 0.0f) || !std::isfinite(p->softcap)) return fail(MXFA_ERR_INVALID_ARG, "softcap must be finite and >= 0");
  if (p->v_fmt != MXFA_FMT_E4M3 && p->v_fmt != MXFA_FMT_E3M2 && p->v_fmt != MXFA_FMT_E3M2_BLK)
    return fail(MXFA_ERR_INVALID_ARG, "v_fmt must be E4M3, E3M2 or E3M2_BLK");
  if (p->block_n != 0 && p->block_n != 64) return fail(MXFA_ERR_UNSUPPORTED, "block_n must be 0 (default) or 64");
  if (p->p_rule != MXFA_P_R1 && p->p_rule != MXFA_P_R2) return fail(MXFA_ERR_INVALID_ARG, "p_rule must be R1 or R2");
  if (p->kv_stride != 0 && (p->kv_stride < p->seq_k || p->kv_stride % 32))
    return fail(MXFA_ERR_INVALID_ARG, "kv_stride must be 0 or a multiple of 32 that is >= seq_k");
  if (decode) {
    if (p->seq_q != 1) return fail(MXFA_ERR_INVALID_ARG, "decode needs seq_q == 1");
    if (p->num_q_heads / p->num_kv_heads > 32)
      return fail(MXFA_ERR_UNSUPPORTED, "decode supports at most 32 query heads per KV head");
  }
  // Per (batch, KV head) the kernels address K/V (and the workspace's bf16 K, 2 bytes per
  // element) through buffer resources of seq_k * 2 * head_dim bytes with 32-bit signed byte
  // offsets: keep that range below 2^31.
  if ((int64_t)p->seq_k * 2 * p->head_dim > (int64_t)INT32_MAX)
    return fail(MXFA_ERR_UNSUPPORTED, "seq_k * head_dim exceeds the kernels' 32-bit K/V range (2^30 elements per head)");
  int64_t qelems = (int64_t)p->batch * p->num_q_heads * p->seq_q * p->head_dim;
  int64_t kelems = (int64_t)p->batch * p->num_kv_heads * (p->kv_stride ? p->kv_stride : p->seq_k) * p->head_dim;
  if (qelems > (int64_t)1 << 40 || kelems > (int64_t)1 << 40) return fail(MXFA_ERR_INVALID_ARG, "tensor too large");
  return MXFA_OK;
}

mxfa_status check_ptrs(const void* const* ptrs, int n) {
  for (int i = 0; i < n; i++) {
    if (!ptrs[i]) return fail(MXFA_ERR_INVALID_ARG, "NULL tensor pointer");
    if (!aligned16(ptrs[i])) return fail(MXFA_ERR_INVALID_ARG, "tensor pointers must be 16-byte aligned");
  }
  return MXFA_OK;
}

FaArgs make_args(const mxfa_attn_params* p, const uint8_t* q, const uint8_t* qs, const uint8_t* k, const uint8_t* ks,
                 const uint8_t* v, const uint8_t* vs, float* o) {
  FaArgs a;
  std::memset(&a, 0, sizeof a);
  a.q = q; a.qs = qs; a.k = k; a.ks = ks; a.v = v; a.vs = vs; a.o = o;
  a.B = p->batch; a.Hq = p->num_q_heads; a.Hkv = p->num_kv_heads; a.Sq = p->seq_q; a.Sk = p->seq_k;
  a.Skc = p->kv_stride ? p->kv_stride : p->seq_k;
  a.q_pos0 = p->q_pos0; a.window = p->window; a.causal = p->causal ? 1 : 0; a.v_e3m2 = p->v_fmt == MXFA_FMT_E3M2;
  a.group = p->num_q_heads / p->num_kv_heads;
  const float log2e = 1.4426950408889634f;
  a.c_log2 = p->softmax_scale * log2e;
  if (p->softcap > 0.0f) {
    a.sc_u = p->softmax_scale / p->softcap;
    a.cap_log2 = p->softcap * log2e;
  }
  return a;
}

// Kernel name for a parameter set; v_suffix adds the V-format suffix of the prefill kernels
// ("_e3m2": E3M2 codes rewritten in LDS, "_blk": block-packed E3M2 read as fp6).
const char* kernel_name(const char* kind, const mxfa_attn_params* p, bool v_suffix = false) {
  static thread_local char buf[64];
  const char* vs = !v_suffix ? "" : p->v_fmt == MXFA_FMT_E3M2 ? "_e3m2" : p->v_fmt == MXFA_FMT_E3M2_BLK ? "_blk" : "";
  std::snprintf(buf, sizeof buf, "mxfa_%s_d%d%s%s%s", kind, p->head_dim, p->softcap > 0.0f ? "_softcap" : "",
                p->p_rule == MXFA_P_R2 ? "_r2" : "", vs);
  return buf;
}

// Split-KV plan: the 64-key blocks of each (b, KV head) are dealt to n_parts interleaved
// partials (partial i: blocks i, i + n_parts, ...), one wave each, about kDecodeWaves
// partial waves per call -- two per SIMD of the 256-CU chip, at the two workgroups per CU
// of D <= 128; half as many at D = 256, whose kernel fits one workgroup per CU (measured
// on B32 Hq16 Hkv8 L8192 D256: 0.169 ms at 1,024 waves, 0.182 at 2,048).  At most 4 partials are
// rounded up to 1, 2 or 4 so that a head's partials fill whole 4-wave workgroups and merge
// inside them.  Interleaving puts the partial waves of a head, which share a workgroup,
// on adjacent blocks at the same time (measured on c5: 188 us vs 204 us for contiguous
// chunks at 2048 waves).  MXFA_DECODE_WAVES overrides the target.
constexpr int64_t kDecodeWaves = 2048;

int64_t decode_wave_target(int head_dim) {
  if (const char* env = getenv("MXFA_DECODE_WAVES")) {
    long long v = atoll(env);
    if (v > 0) return v;
  }
  return head_dim == 256 ? kDecodeWaves / 2 : kDecodeWaves;
}

int decode_parts(const mxfa_attn_params* p) {
  const int64_t bk = (int64_t)p->batch * p->num_kv_heads;
  const int64_t blocks = (p->seq_k + 63) / 64;
  int64_t n = (decode_wave_target(p->head_dim) + bk - 1) / bk;
  if (n == 3) n = 4;
  if (n > blocks) n = blocks;
  if (n < 1) n = 1;
  return (int)n;
}

}  // namespace

extern "C" {

int32_t mxfa_version(void) { return MXFA_VERSION; }

const char* mxfa_status_string(mxfa_status st) {
  switch (st) {
    case MXFA_OK: return "ok";
    case MXFA_ERR_INVALID_ARG: return "invalid argument";
    case MXFA_ERR_UNSUPPORTED: return "unsupported";
    case MXFA_ERR_HIP: return "HIP error";
    case MXFA_ERR_MODULE: return "code object error";
    case MXFA_ERR_WORKSPACE: return "workspace too small";
  }
  return "unknown status";
}

const char* mxfa_last_error(void) { return g_err.c_str(); }

mxfa_status mxfa_init(void) {
  DeviceModule* dm;
  return module_for_current(&dm);
}

void mxfa_shutdown(void) {
  std::lock_guard<std::mutex> lk(g_mu);
  for (auto& kv : g_mods) (void)hipModuleUnload(kv.second.mod);
  g_mods.clear();
}

mxfa_status mxfa_quantize_rows(const float* x, int64_t rows, int32_t cols, mxfa_fmt fmt, uint8_t* codes,
                               uint8_t* scales, void* stream) {
  if (rows < 0 || cols <= 0 || cols % 32) return fail(MXFA_ERR_INVALID_ARG, "cols must be a positive multiple of 32");
  if (fmt != MXFA_FMT_E4M3 && fmt != MXFA_FMT_E3M2) return fail(MXFA_ERR_INVALID_ARG, "bad fmt");
  if (rows == 0) return MXFA_OK;
  if (!x || !codes || !scales) return fail(MXFA_ERR_INVALID_ARG, "NULL pointer");
  if (!aligned16(x) || (reinterpret_cast<uintptr_t>(codes) & 3u))
    return fail(MXFA_ERR_INVALID_ARG, "x must be 16-byte and codes 4-byte aligned");
  int64_t nblocks = rows * (int64_t)cols / 32;
  int64_t threads = nblocks * 8;
  if (mxfa_status st = check_grid((threads + 255) / 256, 256)) return st;
  DeviceModule* dm;
  if (mxfa_status st = module_for_current(&dm)) return st;
  dim3 grid((unsigned)((threads + 255) / 256));
  void* args[] = {(void*)&x, &nblocks, &codes, &scales};
  return launch(dm, fmt == MXFA_FMT_E4M3 ? "mxfa_quant_rows_e4m3" : "mxfa_quant_rows_e3m2", grid, dim3(256), args, stream);
}

mxfa_status mxfa_quantize_rows_r4(const float* x, int64_t rows, int32_t cols, uint8_t* codes, uint8_t* scales,
                                  void* stream) {
  if (rows < 0 || cols <= 0 || cols % 32) return fail(MXFA_ERR_INVALID_ARG, "cols must be a positive multiple of 32");
  if (rows == 0) return MXFA_OK;
  if (!x || !codes || !scales) return fail(MXFA_ERR_INVALID_ARG, "NULL pointer");
  if (!aligned16(x) || (reinterpret_cast<uintptr_t>(codes) & 3u))
    return fail(MXFA_ERR_INVALID_ARG, "x must be 16-byte and codes 4-byte aligned");
  int64_t nblocks = rows * (int64_t)cols / 32;
  if (mxfa_status st = check_grid((nblocks * 8 + 255) / 256, 256)) return st;
  DeviceModule* dm;
  if (mxfa_status st = module_for_current(&dm)) return st;
  void* args[] = {(void*)&x, &nblocks, &codes, &scales};
  return launch(dm, "mxfa_quant_rows_r4", dim3((unsigned)((nblocks * 8 + 255) / 256)), dim3(256), args, stream);
}

mxfa_status mxfa_quantize_cols(const float* x, int64_t mats, int32_t rows, int32_t cols, mxfa_fmt fmt, uint8_t* codes,
                               uint8_t* scales, void* stream) {
  if (mats < 0 || rows <= 0 || rows % 32 || cols <= 0 || cols % 4)
    return fail(MXFA_ERR_INVALID_ARG, "rows must be a positive multiple of 32 and cols of 4");
  if (fmt != MXFA_FMT_E4M3 && fmt != MXFA_FMT_E3M2 && fmt != MXFA_FMT_E3M2_BLK) return fail(MXFA_ERR_INVALID_ARG, "bad fmt");
  if (mats == 0) return MXFA_OK;
  if (!x || !codes || !scales) return fail(MXFA_ERR_INVALID_ARG, "NULL pointer");
  if (!aligned16(x) || (reinterpret_cast<uintptr_t>(codes) & 3u) || (reinterpret_cast<uintptr_t>(scales) & 3u))
    return fail(MXFA_ERR_INVALID_ARG, "x must be 16-byte, codes and scales 4-byte aligned");
  // one wave per (matrix, 32-row block, 128 columns), four waves per workgroup
  const int64_t units = mats * (rows / 32) * ((cols + 127) / 128);
  if (mxfa_status st = check_grid((units + 3) / 4, 256)) return st;
  DeviceModule* dm;
  if (mxfa_status st = module_for_current(&dm)) return st;
  dim3 grid((unsigned)((units + 3) / 4));
  void* args[] = {(void*)&x, &mats, &rows, &cols, &codes, &scales};
  return launch(dm, fmt == MXFA_FMT_E4M3 ? "mxfa_quant_cols_e4m3" : fmt == MXFA_FMT_E3M2 ? "mxfa_quant_cols_e3m2"
                                                                                        : "mxfa_quant_cols_e3m2_blk",
                grid, dim3(256), args, stream);
}

mxfa_status mxfa_kv_append(const mxfa_kv_params* p, const float* k_new, const float* v_new, int32_t pos0, int32_t n_new,
                           uint8_t* k_cache, uint8_t* k_sc, uint8_t* v_cache, uint8_t* v_sc, float* v_tail,
                           void* stream) {
  if (!p) return fail(MXFA_ERR_INVALID_ARG, "params is NULL");
  if (p->batch < 1 || p->num_kv_heads < 1) return fail(MXFA_ERR_INVALID_ARG, "batch and num_kv_heads must be >= 1");
  if (p->head_dim < 32 || p->head_dim % 32) return fail(MXFA_ERR_INVALID_ARG, "head_dim must be a positive multiple of 32");
  if (p->max_len < 32 || p->max_len % 32) return fail(MXFA_ERR_INVALID_ARG, "max_len must be a positive multiple of 32");
  if (p->v_fmt != MXFA_FMT_E4M3 && p->v_fmt != MXFA_FMT_E3M2 && p->v_fmt != MXFA_FMT_E3M2_BLK)
    return fail(MXFA_ERR_INVALID_ARG, "bad v_fmt");
  if (pos0 < 0 || n_new < 0 || (int64_t)pos0 + n_new > p->max_len)
    return fail(MXFA_ERR_INVALID_ARG, "need 0 <= pos0 and pos0 + n_new <= max_len");
  if (n_new == 0) return MXFA_OK;
  const void* ptrs[] = {k_new, v_new, k_cache, k_sc, v_cache, v_sc, v_tail};
  for (const void* q : ptrs)
    if (!q) return fail(MXFA_ERR_INVALID_ARG, "NULL pointer");
  for (const void* q : ptrs)
    if (!aligned16(q)) return fail(MXFA_ERR_INVALID_ARG, "buffers must be 16-byte aligned");
  const int64_t bk = (int64_t)p->batch * p->num_kv_heads;
  int D = p->head_dim, L = p->max_len, n = n_new, pos = pos0;
  // one launch: K (8 lanes per 32-block) then V (one wave per 32 columns of a touched
  // 32-token block)
  int64_t kblocks = bk * n * (D / 32);
  const int64_t kgroups64 = (kblocks * 8 + 255) / 256;
  const int end = pos0 + n_new;
  int ntouch = (end - 1) / 32 - pos0 / 32 + 1;
  int64_t vunits = bk * ntouch * (D / 32);
  const int64_t vgroups = (vunits + 3) / 4;
  if (mxfa_status st = check_grid(kgroups64 + vgroups, 256)) return st;
  int kgroups = (int)kgroups64;
  if (mxfa_status st = check_grid((bk * 32 * (D / 4) + 255) / 256, 256)) return st;   // the tail update
  DeviceModule* dm;
  if (mxfa_status st = module_for_current(&dm)) return st;
  void* args[] = {(void*)&k_new, (void*)&v_new, &v_tail, &kblocks, &kgroups, &vunits, &ntouch,
                  &n, &L, &D, &pos, &k_cache, &k_sc, &v_cache, &v_sc};
  if (mxfa_status st = launch(dm, p->v_fmt == MXFA_FMT_E4M3   ? "mxfa_kv_append_e4m3"
                                  : p->v_fmt == MXFA_FMT_E3M2 ? "mxfa_kv_append_e3m2"
                                                              : "mxfa_kv_append_e3m2_blk",
                              dim3((unsigned)(kgroups + vgroups)), dim3(256), args, stream))
    return st;
  if (end % 32 == 0 || ntouch == 1) return MXFA_OK;   // no open block, or its tail is already written
  // the block left open after a multi-block append keeps its fp32 values for the next one
  int64_t tthreads = bk * 32 * (D / 4);
  void* ta[] = {(void*)&v_new, &v_tail, &tthreads, &n, &D, &pos};
  return launch(dm, "mxfa_kv_tail_update", dim3((unsigned)((tthreads + 255) / 256)), dim3(256), ta, stream);
}

mxfa_status mxfa_softmax_requant(const float* s, const float* row_max, float c, int64_t rows, int32_t cols,
                                 int32_t p_rule, float* p, uint8_t* codes, uint8_t* scales, float* row_sum,
                                 void* stream) {
  if (rows < 0 || cols <= 0 || cols % 32) return fail(MXFA_ERR_INVALID_ARG, "cols must be a positive multiple of 32");
  if (p_rule != MXFA_P_R1 && p_rule != MXFA_P_R2) return fail(MXFA_ERR_INVALID_ARG, "p_rule must be R1 or R2");
  if (!(c > 0.0f) || !std::isfinite(c)) return fail(MXFA_ERR_INVALID_ARG, "c must be finite and > 0");
  if (rows == 0) return MXFA_OK;
  if (!s || !row_max || !p || !codes || !scales || !row_sum) return fail(MXFA_ERR_INVALID_ARG, "NULL pointer");
  if (!aligned16(s) || (reinterpret_cast<uintptr_t>(codes) & 3u))
    return fail(MXFA_ERR_INVALID_ARG, "s must be 16-byte and codes 4-byte aligned");
  if (mxfa_status st = check_grid((rows + 255) / 256, 256)) return st;
  DeviceModule* dm;
  if (mxfa_status st = module_for_current(&dm)) return st;
  dim3 grid((unsigned)((rows + 255) / 256));
  int cols_i = cols;
  int rule = p_rule;
  void* args[] = {(void*)&s, (void*)&row_max, &c, &rows, &cols_i, &p, &codes, &scales, &row_sum, &rule};
  return launch(dm, "mxfa_softmax_requant_rows", grid, dim3(256), args, stream);
}

mxfa_status mxfa_gemm(const mxfa_gemm_params* p, const uint8_t* a, const uint8_t* a_sc, const uint8_t* b,
                      const uint8_t* b_sc, void* c, void* stream) {
  if (!p) return fail(MXFA_ERR_INVALID_ARG, "params is NULL");
  if (p->m < 1 || p->n < 1 || p->k < 1) return fail(MXFA_ERR_INVALID_ARG, "m, n and k must be >= 1");
  if (p->k % 32) return fail(MXFA_ERR_INVALID_ARG, "k must be a multiple of 32 (scale blocks)");
  if (p->k % 64 || p->m % 16 || p->n % 16)
    return fail(MXFA_ERR_UNSUPPORTED, "mxfa_gemm needs k % 64 == 0, m % 16 == 0 and n % 16 == 0");
  if (p->a_fmt != MXFA_FMT_E4M3 && p->a_fmt != MXFA_FMT_E3M2) return fail(MXFA_ERR_INVALID_ARG, "bad a_fmt");
  if (p->b_fmt != MXFA_FMT_E4M3 && p->b_fmt != MXFA_FMT_E3M2) return fail(MXFA_ERR_INVALID_ARG, "bad b_fmt");
  if (p->c_fmt != MXFA_C_F32 && p->c_fmt != MXFA_C_BF16) return fail(MXFA_ERR_INVALID_ARG, "bad c_fmt");
  const int64_t lim = (int64_t)1 << 31;
  if (p->m * p->k >= lim || p->k * p->n >= lim)
    return fail(MXFA_ERR_UNSUPPORTED, "mxfa_gemm operands are limited to 2^31 elements");
  if (p->n >= ((int64_t)1 << 22))   // a 256-row tile of C stays under 2^32 bytes
    return fail(MXFA_ERR_UNSUPPORTED, "mxfa_gemm needs n < 4194304");
  const void* ptrs[] = {a, a_sc, b, b_sc, c};
  if (mxfa_status st = check_ptrs(ptrs, 5)) return st;
  DeviceModule* dm;
  if (mxfa_status st = module_for_current(&dm)) return st;
  GemmArgs g;
  std::memset(&g, 0, sizeof g);
  g.a = a; g.sa = a_sc; g.b = b; g.sb = b_sc; g.c = static_cast<uint8_t*>(c);
  g.c_bf16 = p->c_fmt == MXFA_C_BF16;
  g.M = (int)p->m; g.N = (int)p->n; g.K = (int)p->k;
  g.a_e3m2 = p->a_fmt == MXFA_FMT_E3M2;
  g.b_e3m2 = p->b_fmt == MXFA_FMT_E3M2;
  static const char* const names[2][2] = {{"mxfa_gemm", "mxfa_gemm_be3m2"},
                                          {"mxfa_gemm_ae3m2", "mxfa_gemm_ae3m2_be3m2"}};
  const int64_t tm = (p->m + 255) / 256, tn = (p->n + 255) / 256;
  g.tiles_n = (int)tn;
  // the kernels are built for one workgroup size (their launch bounds): 256 or 512 threads.
  // E4M3 operands with whole K steps (k % 128 == 0) take the LDS-DMA kernel
  // (MXFA_GEMM=reg selects the register-staged one, for comparison).
  const char* sel = getenv("MXFA_GEMM");
  // M <= 128 with E4M3 operands (the batched-decode projection): the skinny kernel, one
  // workgroup per 32-column strip (MXFA_GEMM=big or =reg selects the tiled kernels instead)
  // (its LDS holds all of SA and the strip's SB: (k / 32) (m + 32) <= 96 KiB)
  if (!g.a_e3m2 && !g.b_e3m2 && p->m <= 128 && (p->k / 32) * (p->m + 32) <= 96 * 1024 &&
      !(sel && (std::strcmp(sel, "big") == 0 || std::strcmp(sel, "reg") == 0))) {
    const char* sk = p->m <= 32 ? "mxfa_gemm_skinny_t1" : p->m <= 64 ? "mxfa_gemm_skinny_t2" : "mxfa_gemm_skinny_t4";
    void* args[] = {&g};
    return launch(dm, sk, dim3((unsigned)((p->n + 31) / 32)), dim3(256), args, stream);
  }
  const bool dma = !g.a_e3m2 && !g.b_e3m2 && p->k % 128 == 0 && !(sel && std::strcmp(sel, "reg") == 0);
  const char* name = dma ? "mxfa_gemm_dma" : names[g.a_e3m2][g.b_e3m2];
  int threads = 0;
  MXFA_HIP(hipFuncGetAttribute(&threads, HIP_FUNC_ATTRIBUTE_MAX_THREADS_PER_BLOCK, fn_by_name(dm, name)));
  if (threads != 256 && threads != 512)
    return fail(MXFA_ERR_MODULE, std::string(name) + " has an unexpected workgroup size " + std::to_string(threads));
  void* args[] = {&g};
  return launch(dm, name, dim3((unsigned)(tm * tn)), dim3((unsigned)threads), args, stream);
}

mxfa_status mxfa_fill_normal(float* x, int64_t n, uint64_t seed, float outlier_p, float outlier_mul, void* stream) {
  if (n < 0) return fail(MXFA_ERR_INVALID_ARG, "n must be >= 0");
  if (n == 0) return MXFA_OK;
  if (!x) return fail(MXFA_ERR_INVALID_ARG, "NULL pointer");
  if (mxfa_status st = check_grid((n + 255) / 256, 256)) return st;
  DeviceModule* dm;
  if (mxfa_status st = module_for_current(&dm)) return st;
  dim3 grid((unsigned)((n + 255) / 256));
  void* args[] = {&x, &n, &seed, &outlier_p, &outlier_mul};
  return launch(dm, "mxfa_fill_normal_f32", grid, dim3(256), args, stream);
}

}  // extern "C"

namespace {
// Workgroup shape of the prefill kernels: nw waves, hpw query heads (of one KV head) per
// workgroup, nw / hpw 32-query waves each.
FaArgs prefill_args(const mxfa_attn_params* p, const uint8_t* q, const uint8_t* q_sc, const uint8_t* k,
                    const uint8_t* k_sc, const uint8_t* v, const uint8_t* v_sc, float* o, int nw, dim3& grid) {
  FaArgs a = make_args(p, q, q_sc, k, k_sc, v, v_sc, o);
  a.hpw = 1;
  for (int h = nw; h > 1; h /= 2)
    if (a.group % h == 0) {
      a.hpw = h;
      break;
    }
  a.qpw = 32 * (nw / a.hpw);
  a.n_qblk = (p->seq_q + a.qpw - 1) / a.qpw;
  grid = dim3((unsigned)a.n_qblk, (unsigned)(p->batch * p->num_kv_heads * (a.group / a.hpw)));
  return a;
}

// Wave-blocks (32 queries x 64 keys) of one launch of the prefill3 grid: every wave of a
// workgroup walks the workgroup's key blocks [j0, j1) (the kernels' own loop bounds).
int64_t prefill3_wave_blocks(const FaArgs& a, const mxfa_attn_params* p) {
  const int nkb = (p->seq_k + 63) / 64;
  int64_t per_group = 0;
  for (int qblk = 0; qblk < a.n_qblk; qblk++) {
    const int q0 = qblk * a.qpw, qmax = std::min(q0 + a.qpw, p->seq_q) - 1;
    const int j0 = p->window > 0 ? std::max(0, p->q_pos0 + q0 - p->window + 1) / 64 : 0;
    const int j1 = p->causal ? std::min(nkb, std::max(0, p->q_pos0 + qmax) / 64 + 1) : nkb;
    per_group += 4 * std::max(0, j1 - j0);
  }
  return per_group * p->batch * p->num_kv_heads * (a.group / a.hpw);
}

// mxfa_prefill_ws widens K to bf16 once, into the workspace, by a pre-pass -- or leaves it to
// the workspace-free kernel, whose workgroups widen each block they read in LDS: each K
// element about 16 * wave_blocks / (B * Hkv * Sk) times.  Measured (same box): at 8.5 (MHA,
// S = 2048) the in-LDS form is 3.4% faster; at 49 (Gemma shape) 2-4% and at 65 (GQA-4, S =
// 4096) 6.5% slower.  Below 32 the call runs the workspace-free kernel (the workspace is
// then not touched).
bool prefill_ws_widens_in_lds(const FaArgs& a, const mxfa_attn_params* p) {
  return 16 * prefill3_wave_blocks(a, p) < (int64_t)32 * p->batch * p->num_kv_heads * p->seq_k;
}

// Waves per workgroup of the workspace kernel (mxfa_prefill3_*).
int prefill3_waves(const mxfa_attn_params*) { return 4; }

// Workspace of mxfa_prefill_ws: the bf16 copy of K, then (E3M2 V) the E4M3 copy of V.
size_t prefill3_kbf_bytes(const mxfa_attn_params* p) {
  return (size_t)p->batch * p->num_kv_heads * p->seq_k * p->head_dim * 2;
}
size_t prefill3_workspace(const mxfa_attn_params* p) {
  const size_t v = p->v_fmt == MXFA_FMT_E3M2 ? (size_t)p->batch * p->num_kv_heads * p->seq_k * p->head_dim : 0;
  return prefill3_kbf_bytes(p) + v;
}

}  // namespace

extern "C" {

mxfa_status mxfa_prefill(const mxfa_attn_params* p, const uint8_t* q, const uint8_t* q_sc, const uint8_t* k,
                         const uint8_t* k_sc, const uint8_t* v, const uint8_t* v_sc, float* o, void* stream) {
  if (mxfa_status st = check_params(p, false)) return st;
  const void* ptrs[] = {q, q_sc, k, k_sc, v, v_sc, o};
  if (mxfa_status st = check_ptrs(ptrs, 7)) return st;
  DeviceModule* dm;
  if (mxfa_status st = module_for_current(&dm)) return st;
  dim3 grid;
  FaArgs a = prefill_args(p, q, q_sc, k, k_sc, v, v_sc, o, 4, grid);
  void* args[] = {&a};
  // the workspace kernel's design in its workspace-free form: K widened to bf16 in LDS, E3M2
  // V read as E5M2
  return launch(dm, kernel_name("prefill3n", p, true), grid, dim3(256), args, stream);
}

mxfa_status mxfa_prefill_plan(const mxfa_attn_params* p, size_t* workspace_bytes) {
  if (mxfa_status st = check_params(p, false)) return st;
  if (!workspace_bytes) return fail(MXFA_ERR_INVALID_ARG, "workspace_bytes is NULL");
  *workspace_bytes = prefill3_workspace(p);
  return MXFA_OK;
}

}  // extern "C"

namespace {
// The workspace prefill (mxfa_prefill_ws), or with tr set its stage trace: the one
// workgroup that holds query rows 32 * tr->q_tile .. + 31 of head tr->bh.
struct TraceReq {
  int32_t bh, q_tile;
  float *s_out, *ml_out;
  uint8_t *p_out, *ps_out;
};

mxfa_status prefill_ws_impl(const mxfa_attn_params* p, const uint8_t* q, const uint8_t* q_sc, const uint8_t* k,
                            const uint8_t* k_sc, const uint8_t* v, const uint8_t* v_sc, float* o, void* workspace,
                            size_t workspace_bytes, void* stream, const TraceReq* tr) {
  const void* ptrs[] = {q, q_sc, k, k_sc, v, v_sc, o};
  if (mxfa_status st = check_ptrs(ptrs, 7)) return st;
  const size_t need = prefill3_workspace(p);
  if (!workspace || workspace_bytes < need)
    return fail(MXFA_ERR_WORKSPACE, "prefill workspace needs " + std::to_string(need) + " bytes");
  if (!aligned16(workspace)) return fail(MXFA_ERR_INVALID_ARG, "workspace must be 16-byte aligned");
  DeviceModule* dm;
  if (mxfa_status st = module_for_current(&dm)) return st;
  const int nw = prefill3_waves(p);
  dim3 grid;
  FaArgs a = prefill_args(p, q, q_sc, k, k_sc, v, v_sc, o, nw, grid);
  if (!tr && prefill_ws_widens_in_lds(a, p)) {
    void* args[] = {&a};
    return launch(dm, kernel_name("prefill3n", p, true), grid, dim3(256), args, stream);
  }
  uint8_t* kbf = static_cast<uint8_t*>(workspace);
  // (E3M2 V codes one per byte: widened to E4M3 by the pre-pass; block-packed E3M2 V is read
  // by the kernel as it is)
  uint8_t* vws = p->v_fmt == MXFA_FMT_E3M2 ? kbf + prefill3_kbf_bytes(p) : nullptr;
  a.kbf = kbf;
  a.vws = vws;
  // bf16 K (and E4M3 V) in one launch: 16 pieces of 8 codes per thread, one (batch, KV head)
  // per grid row
  int D = p->head_dim, Sk = p->seq_k, Skc = a.Skc;
  const int64_t pieces = (int64_t)Sk * (D / 8);    // per (batch, KV head)
  if (pieces > INT32_MAX - 256 * 16) return fail(MXFA_ERR_UNSUPPORTED, "seq_k * head_dim / 8 exceeds the workspace pre-pass's range");
  const dim3 cgrid((unsigned)((pieces + 256 * 16 - 1) / (256 * 16)), (unsigned)(p->batch * p->num_kv_heads));
  void* cargs[] = {(void*)&k, (void*)&k_sc, (void*)&v, &D, &Sk, &Skc, &kbf, &vws};
  if (mxfa_status st = launch(dm, "mxfa_k_to_bf16", cgrid, dim3(256), cargs, stream)) return st;
  void* args[] = {&a};
  if (!tr) return launch(dm, kernel_name("prefill3", p, p->v_fmt == MXFA_FMT_E3M2_BLK), grid, dim3((unsigned)(64 * nw)),
                         args, stream);
  // the item (qx, qy) of the traced rows, as the kernel's own mapping assigns them
  const int b = tr->bh / p->num_q_heads, head = tr->bh % p->num_q_heads;
  const int kvh = head / a.group, hc = (head % a.group) / a.hpw;
  const int qblk = 32 * tr->q_tile / a.qpw;
  a.tr_qy = (b * p->num_kv_heads + kvh) * (a.group / a.hpw) + hc;
  a.tr_qx = p->causal ? a.n_qblk - 1 - qblk : qblk;
  a.tr_head = head;
  a.tr_q0 = 32 * tr->q_tile;
  a.tr_s = tr->s_out;
  a.tr_ml = tr->ml_out;
  a.tr_p = tr->p_out;
  a.tr_ps = tr->ps_out;
  return launch(dm, kernel_name("prefill3_trace", p), dim3(1), dim3((unsigned)(64 * nw)), args, stream);
}
}  // namespace

extern "C" {

mxfa_status mxfa_prefill_ws(const mxfa_attn_params* p, const uint8_t* q, const uint8_t* q_sc, const uint8_t* k,
                            const uint8_t* k_sc, const uint8_t* v, const uint8_t* v_sc, float* o, void* workspace,
                            size_t workspace_bytes, void* stream) {
  if (mxfa_status st = check_params(p, false)) return st;
  return prefill_ws_impl(p, q, q_sc, k, k_sc, v, v_sc, o, workspace, workspace_bytes, stream, nullptr);
}

mxfa_status mxfa_prefill_trace(const mxfa_attn_params* p, const uint8_t* q, const uint8_t* q_sc, const uint8_t* k,
                               const uint8_t* k_sc, const uint8_t* v, const uint8_t* v_sc, float* o,
                               void* workspace, size_t workspace_bytes, int32_t bh, int32_t q_tile, float* s_out,
                               float* ml_out, uint8_t* p_out, uint8_t* ps_out, void* stream) {
  if (mxfa_status st = check_params(p, false)) return st;
  if (bh < 0 || bh >= p->batch * p->num_q_heads || q_tile < 0 || 32 * q_tile >= p->seq_q)
    return fail(MXFA_ERR_INVALID_ARG, "bh or q_tile out of range");
  if (!s_out || !ml_out || !p_out || !ps_out) return fail(MXFA_ERR_INVALID_ARG, "NULL trace buffer");
  if (p->v_fmt == MXFA_FMT_E3M2_BLK) return fail(MXFA_ERR_UNSUPPORTED, "the stage trace reads V as E4M3 or E3M2 codes");
  const TraceReq tr = {bh, q_tile, s_out, ml_out, p_out, ps_out};
  return prefill_ws_impl(p, q, q_sc, k, k_sc, v, v_sc, o, workspace, workspace_bytes, stream, &tr);
}

mxfa_status mxfa_decode_plan(const mxfa_attn_params* p, int32_t* n_parts, size_t* workspace_bytes) {
  if (mxfa_status st = check_params(p, true)) return st;
  const int np = decode_parts(p);
  if (n_parts) *n_parts = np;
  if (workspace_bytes)
    *workspace_bytes = (size_t)p->batch * p->num_q_heads * np * (p->head_dim + 2) * sizeof(float) + 256;
  return MXFA_OK;
}

}  // extern "C"

namespace {

// The decode launches of mxfa_decode and mxfa_decode_noalloc (arguments already checked;
// workspace holds the partials of the two-launch path).
mxfa_status decode_launch(DeviceModule* dm, const mxfa_attn_params* p, const uint8_t* q, const uint8_t* q_sc,
                          const uint8_t* k_cache, const uint8_t* k_sc, const uint8_t* v_cache, const uint8_t* v_sc,
                          float* o, void* workspace, void* stream) {
  FaArgs a = make_args(p, q, q_sc, k_cache, k_sc, v_cache, v_sc, o);
  const int nparts = decode_parts(p);
  a.n_qblk = nparts;
  int64_t nbh = (int64_t)p->batch * p->num_q_heads;
  a.part_o = reinterpret_cast<float*>(workspace);
  a.part_ml = a.part_o + nbh * nparts * p->head_dim;
  // 4 waves per workgroup over the linear (b, KV head, chunk) items
  const int nw = 4;
  const int64_t items = (int64_t)p->batch * p->num_kv_heads * nparts;
  const dim3 grid((unsigned)((items + nw - 1) / nw));
  // When every head's partials fit in one workgroup (nparts divides its 4 waves) and the
  // valid columns' partials fit the waves' V slots (group <= 16), the kernel merges them
  // itself (same formula and order as mxfa_decode_combine) and no combine launch follows.
  // MXFA_DECODE_COMBINE=kernel selects the combine kernel always (the two paths give
  // bit-identical O; the switch exists to test exactly that).
  const char* comb = getenv("MXFA_DECODE_COMBINE");
  const bool force_kernel = comb && std::strcmp(comb, "kernel") == 0;
  a.fuse_combine = !force_kernel && nw % nparts == 0 && a.group <= 16;
  void* args[] = {&a};
  if (mxfa_status st = launch(dm, kernel_name("decode", p, p->v_fmt == MXFA_FMT_E3M2_BLK), grid, dim3(64 * nw), args,
                              stream))
    return st;
  if (a.fuse_combine) return MXFA_OK;
  return launch(dm, "mxfa_decode_combine", dim3((unsigned)nbh), dim3((unsigned)p->head_dim), args, stream);
}

}  // namespace

extern "C" {

mxfa_status mxfa_decode(const mxfa_attn_params* p, const uint8_t* q, const uint8_t* q_sc, const uint8_t* k_cache,
                        const uint8_t* k_sc, const uint8_t* v_cache, const uint8_t* v_sc, float* o, void* workspace,
                        size_t workspace_bytes, void* stream) {
  if (mxfa_status st = check_params(p, true)) return st;
  const void* ptrs[] = {q, q_sc, k_cache, k_sc, v_cache, v_sc, o};
  if (mxfa_status st = check_ptrs(ptrs, 7)) return st;
  size_t need = 0;
  int32_t sl = 0;
  mxfa_decode_plan(p, &sl, &need);
  if (!workspace || workspace_bytes < need)
    return fail(MXFA_ERR_WORKSPACE, "decode workspace must be at least " + std::to_string(need) + " bytes");
  if (!aligned16(workspace)) return fail(MXFA_ERR_INVALID_ARG, "workspace must be 16-byte aligned");
  DeviceModule* dm;
  if (mxfa_status st = module_for_current(&dm)) return st;
  return decode_launch(dm, p, q, q_sc, k_cache, k_sc, v_cache, v_sc, o, workspace, stream);
}

mxfa_status mxfa_decode_noalloc(const mxfa_attn_params* p, const uint8_t* q, const uint8_t* q_sc,
                                const uint8_t* k_cache, const uint8_t* k_sc, const uint8_t* v_cache,
                                const uint8_t* v_sc, float* o, void* stream) {
  if (mxfa_status st = check_params(p, true)) return st;
  const void* ptrs[] = {q, q_sc, k_cache, k_sc, v_cache, v_sc, o};
  if (mxfa_status st = check_ptrs(ptrs, 7)) return st;
  size_t need = 0;
  int32_t sl = 0;
  mxfa_decode_plan(p, &sl, &need);
  if (need > MXFA_DECODE_SCRATCH_BYTES)
    return fail(MXFA_ERR_WORKSPACE, "mxfa_decode_noalloc: the partials of this shape need " + std::to_string(need) +
                                        " bytes, above the " + std::to_string(MXFA_DECODE_SCRATCH_BYTES) +
                                        "-byte device scratch; use mxfa_decode with a workspace");
  DeviceModule* dm;
  if (mxfa_status st = loaded_module_for_current(&dm)) return st;
  return decode_launch(dm, p, q, q_sc, k_cache, k_sc, v_cache, v_sc, o, dm->decode_scratch, stream);
}

}  // extern "C"
