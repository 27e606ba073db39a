// C ABI of libtexelator_hip.so: handle ownership, upload/repack, dispatch, diagnostics.
//
// Reference counterparts (texelator/cuda/texelator_cuda.cu): Handle :47-73, pack :1260-1327,
// dispatch :1329-1469, setters :1471-1503, handle_info :1505-1512, free :1538, probe :1551-1595.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstring>
#include <mutex>
#include <new>
#include <string>
#include <thread>
#include <vector>

#include "../../include/texelator_hip.h"
#include "bc4_device.h"
#include "elementwise.h"
#include "kernels.h"

// Static scratch of tx_linear_noalloc: split-K partial sums for callers that cannot allocate.
// File-scope device memory: every GPU the library runs on holds its own copy from the first use
// until the process ends. In host code `scratch` is only a stand-in symbol; its device address on
// each GPU comes from hipGetSymbolAddress (with that GPU current) and is the only form ever passed
// to a kernel. 32 MiB holds every prefill split this library chooses (prefill_splits caps the
// partials at 32 MiB) and the one-token GEMV splits of any matrix up to ~1M output rows.
constexpr size_t kScratchBytes = size_t(32) << 20;
static __device__ __align__(256) float scratch[kScratchBytes / sizeof(float)];

namespace {

thread_local std::string g_last_error;

int fail(int code, const std::string &message) {
  g_last_error = message;
  return code;
}

#define TX_HIP(call)                                                                   \
  do {                                                                                 \
    hipError_t _e = (call);                                                            \
    if (_e != hipSuccess) return fail(TX_ERR_HIP, std::string("HIP: ") + hipGetErrorString(_e) + " (" #call ")"); \
  } while (0)

struct DeviceGuard {
  int previous = -1;
  bool changed = false;
  explicit DeviceGuard(int device) {
    if (hipGetDevice(&previous) == hipSuccess && previous != device) changed = hipSetDevice(device) == hipSuccess;
  }
  ~DeviceGuard() {
    if (changed) (void)hipSetDevice(previous);
  }
};

constexpr uint32_t kHandleMagic = 0x54584834u;  // "TXH4"

struct Handle {
  uint32_t magic = kHandleMagic;
  int M = 0, K = 0, bpr = 0, Mp = 0, bp = 0, RG = 0, CG = 0, device = 0;
  int lookahead = 1;
  int prefill_threshold = 16, prefill_tile_rows = 1024, prefill_backend = 0;
  int gemv_splits = 1;
  int cus = 256;
  uint4 *tiles = nullptr;
  float *scales = nullptr;
  void *bias = nullptr;
  int bias_dtype = -1;
  float *partials = nullptr;
  const float4 *lut = nullptr;  // LUT mode: caller-owned 255 x 255 x 8 fp32 device palette table

  ~Handle() {
    DeviceGuard guard(device);
    if (tiles) (void)hipFree(tiles);
    if (scales) (void)hipFree(scales);
    if (bias) (void)hipFree(bias);
    if (partials) (void)hipFree(partials);
    magic = 0;
  }
};

Handle *as_handle(uint64_t value) {
  auto *h = reinterpret_cast<Handle *>(value);
  if (!h || h->magic != kHandleMagic) return nullptr;
  return h;
}

void repack_rows(const uint8_t *blocks, const Handle &h, uint32_t *out, int g_begin, int g_end) {
  for (int g = g_begin; g < g_end; ++g) {
    for (int c = 0; c < h.CG; ++c) {
      uint32_t *tile = out + ((size_t)g * h.CG + c) * 256;
      for (int lane = 0; lane < 64; ++lane) {
        const int m = g * tx::kTileRows + (lane & 15);
        for (int half = 0; half < 2; ++half) {
          const int blk = c * tx::kTileBlocks + 2 * (lane >> 4) + half;
          uint32_t a = tx::kZeroBlockWord, b = tx::kZeroBlockWord;
          if (m < h.M && blk < h.bpr) tx::encode_device_block(blocks + ((size_t)m * h.bpr + blk) * 8, a, b);
          tile[lane * 4 + half * 2] = a;
          tile[lane * 4 + half * 2 + 1] = b;
        }
      }
    }
  }
}

// K splits of the single-token GEMV. Tall matrices (>= 1024 row groups) fill the chip without
// splitting; shorter ones split K so that there are about TX_GEMV_SPLIT_TARGET workgroups per CU
// (TX_GEMV_SPLIT_TARGET_SHORT_K where K is at most 64 tile columns), each covering at least 4
// tile columns. A split never covers more tile columns than the LDS x slice holds.
int device_cus(int device) {
  hipDeviceProp_t prop;
  if (hipGetDeviceProperties(&prop, device) == hipSuccess && prop.multiProcessorCount > 0) return prop.multiProcessorCount;
  return 256;
}

// Target workgroups per CU for short matrices (their one-token GEMV is latency-bound).
#ifndef TX_GEMV_SPLIT_TARGET
#define TX_GEMV_SPLIT_TARGET 4
#endif
#ifndef TX_GEMV_SPLIT_TARGET_SHORT_K
#define TX_GEMV_SPLIT_TARGET_SHORT_K TX_GEMV_SPLIT_TARGET
#endif

int choose_splits(int RG, int CG, int cus) {
  int ks = 1;
  if (RG < 1024) {
    const int target = CG <= 64 ? TX_GEMV_SPLIT_TARGET_SHORT_K : TX_GEMV_SPLIT_TARGET;
    ks = (target * cus + RG - 1) / RG;
    ks = std::min(ks, std::max(1, CG / 4));
  }
  ks = std::max(ks, (CG + tx::kGemvMaxLdsColumns - 1) / tx::kGemvMaxLdsColumns);
  ks = std::min(ks, std::max(1, 0x7FFFFFFF / std::max(CG, 1)));  // the kernel's 32-bit split arithmetic
  return std::max(1, std::min(ks, CG));
}

// Workspace bytes of a prefill call (split-K partials), 0 if none.
int64_t prefill_workspace_bytes(const Handle *h, int64_t tokens) {
  const int ks = tx::prefill_splits(h->M, h->CG, tokens, h->cus);
  return ks > 1 ? (int64_t)ks * tokens * h->Mp * (int64_t)sizeof(float) : 0;
}

// The dense-scratch backend (the reference's backend 1, texelator_cuda.cu:937-990): its scratch
// holds min(tile_rows, M) decoded rows of K 16-bit weights, then the library GEMM's workspace.
constexpr int kDenseBackend = 1;

int dense_tile_rows(const Handle *h) { return std::min(h->prefill_tile_rows, h->M); }

int64_t dense_rows_bytes(const Handle *h) { return ((int64_t)dense_tile_rows(h) * h->K * 2 + 255) / 256 * 256; }

// The library GEMM's workspace starts at the first 256-byte boundary after the decoded rows (the
// caller's workspace need only be 16-byte aligned): 256 bytes of slack cover the alignment.
int64_t dense_workspace_bytes(const Handle *h) { return dense_rows_bytes(h) + 256 + (int64_t)tx::kDenseGemmWorkspace; }

// The backend a prefill-sized call of `tokens` tokens runs: the dense-scratch path, or a tile id.
int prefill_choice(const Handle *h, int64_t tokens) {
  if (h->prefill_backend == kDenseBackend) return kDenseBackend;
  return h->prefill_backend >= tx::kPrefillFirst ? h->prefill_backend
                                                 : tx::prefill_default_candidate(h->M, h->K, tokens, h->cus);
}

// Workspace bytes of a prefill-sized call.
int64_t prefill_call_bytes(const Handle *h, int64_t tokens) {
  return prefill_choice(h, tokens) == kDenseBackend ? dense_workspace_bytes(h) : prefill_workspace_bytes(h, tokens);
}

// Rows decoded tile_rows at a time into the workspace, one hipBLASLt GEMM per row tile writing
// its columns of y, then the bias with a second rounding (texelator_cuda.cu:960-989).
int run_dense_prefill(Handle *h, const void *x, bool f16, int64_t tokens, void *y, void *workspace,
                      int64_t workspace_bytes, hipStream_t stream) {
  if (tokens > (1 << 20)) return fail(TX_ERR_INVALID, "token count exceeds the prefill limit (1048576)");
  if (!workspace || workspace_bytes < dense_workspace_bytes(h) || reinterpret_cast<uintptr_t>(workspace) % 16 != 0)
    return fail(TX_ERR_INVALID, "dense prefill workspace missing or too small (see tx_workspace_bytes)");
  uint16_t *dense = static_cast<uint16_t *>(workspace);
  const uintptr_t rows_end = reinterpret_cast<uintptr_t>(workspace) + (uintptr_t)dense_rows_bytes(h);
  void *gemm_workspace = reinterpret_cast<void *>((rows_end + 255) & ~uintptr_t(255));
  const int tile = dense_tile_rows(h);
  for (int row = 0; row < h->M; row += tile) {
    const int rows = std::min(tile, h->M - row);
    TX_HIP(tx::launch_decode_rows(h->tiles, h->scales, h->lut, h->M, h->K, h->CG, row, rows, f16, dense, stream));
    std::string error;
    if (!tx::dense_gemm(h->device, f16, rows, tokens, h->K, dense, x, static_cast<uint16_t *>(y) + row, h->M,
                        gemm_workspace, stream, error))
      return fail(TX_ERR_HIP, "dense prefill: " + error);
  }
  if (h->bias) TX_HIP(tx::launch_add_bias(y, h->bias, tokens, h->M, f16, stream));
  return TX_OK;
}

int run_prefill(Handle *h, int candidate, const void *x, bool f16, int64_t tokens, void *y, void *workspace,
                int64_t workspace_bytes, hipStream_t stream) {
  if (candidate == kDenseBackend) return run_dense_prefill(h, x, f16, tokens, y, workspace, workspace_bytes, stream);
  tx::PrefillParams p{};
  p.f16 = f16 ? 1 : 0;
  p.lut = h->lut;
  p.tiles = h->tiles;
  p.scales = h->scales;
  p.x = x;
  p.bias = h->bias;
  p.y = y;
  p.M = h->M;
  p.K = h->K;
  p.Mp = h->Mp;
  p.RG = h->RG;
  p.CG = h->CG;
  p.tokens = (int)tokens;
  p.ks = tx::prefill_splits(h->M, h->CG, tokens, h->cus);
  if (tokens > (1 << 20)) return fail(TX_ERR_INVALID, "token count exceeds the prefill limit (1048576)");
  const int64_t need = prefill_workspace_bytes(h, tokens);
  if (need > 0) {
    if (!workspace || workspace_bytes < need || reinterpret_cast<uintptr_t>(workspace) % 16 != 0)
      return fail(TX_ERR_INVALID, "prefill workspace missing or too small (see tx_workspace_bytes)");
    p.partials = static_cast<float *>(workspace);
  }
  TX_HIP(tx::launch_prefill(p, candidate, stream));
  return TX_OK;
}

// The single-token split-K partials a handle's last tx_linear_split wrote.
// Heads times chunks up to which an o GEMV workgroup merges the attention partials itself (the
// merge reads that many 520-byte rows per workgroup).
constexpr int kMergeMaxChunkHeads = 64;

tx::SplitSource split_source(const Handle *h) {
  return tx::SplitSource{h->partials, static_cast<const uint16_t *>(h->bias), h->gemv_splits, h->Mp, 1};
}

// One-token K splits write ks * Mp fp32 partials to `partials` (the handle's own buffer, or the
// static scratch of tx_linear_noalloc); several tokens run unsplit and write none.
// One-token calls of this handle run every K split in one workgroup (gemv_fused_kernel).
bool one_token_fused(const Handle *h) {
  return !h->lut && tx::gemv_fused_profitable(h->RG, h->CG, h->gemv_splits, h->cus);
}

int64_t gemv_partials_bytes(const Handle *h, int64_t tokens) {
  if (tokens != 1 || h->gemv_splits == 1 || one_token_fused(h)) return 0;
  return (int64_t)h->gemv_splits * h->Mp * (int64_t)sizeof(float);
}

int run_gemv(Handle *h, const void *x, bool f16, int64_t tokens, void *y, bool f32_out, hipStream_t stream,
             float *partials) {
  if (tokens > 65535) return fail(TX_ERR_INVALID, "token grid exceeds the HIP grid.z limit");
  tx::GemvParams p{};
  p.f16 = f16 ? 1 : 0;
  p.lut = h->lut;
  p.tiles = h->tiles;
  p.scales = h->scales;
  p.x = x;
  p.bias = f32_out ? nullptr : h->bias;
  p.y = y;
  p.M = h->M;
  p.K = h->K;
  p.Mp = h->Mp;
  p.RG = h->RG;
  p.CG = h->CG;
  p.tokens = (int)tokens;
  // One token: K splits reduced by a second kernel. Several tokens: one pass per 16 tokens.
  p.ks = tokens == 1 ? h->gemv_splits : 1;
  p.partials = partials;
  p.fused = tokens == 1 && one_token_fused(h) ? 1 : 0;
  TX_HIP(tx::launch_gemv(p, h->lookahead, f32_out, stream));
  return TX_OK;
}

int run_gemv_split(Handle *h, const void *x, hipStream_t stream) {
  tx::GemvParams p{};
  p.tiles = h->tiles;
  p.scales = h->scales;
  p.x = x;
  p.M = h->M;
  p.K = h->K;
  p.Mp = h->Mp;
  p.RG = h->RG;
  p.CG = h->CG;
  p.tokens = 1;
  p.ks = h->gemv_splits;
  p.partials = h->partials;
  p.force_partials = 1;
  p.lut = h->lut;
  TX_HIP(tx::launch_gemv(p, h->lookahead, true, stream));
  return TX_OK;
}

// Shared by tx_pack_encoded (host blocks and scales) and tx_pack_encoded_device (device ones).
int pack_common(const uint8_t *blocks, int64_t blocks_bytes, const float *scales, int64_t rows, const void *bias,
                int bias_dtype, int device, bool on_device, uint64_t *handle_out) {
  g_last_error.clear();
  if (!blocks || !scales || !handle_out) return fail(TX_ERR_INVALID, "blocks, scales and handle_out must be non-null");
  if (rows <= 0 || blocks_bytes <= 0 || blocks_bytes % (rows * 8) != 0) return fail(TX_ERR_INVALID, "invalid encoded size");
  const int64_t bpr = blocks_bytes / (rows * 8);
  if (rows > (1 << 30) || bpr * 16 > (1 << 30)) return fail(TX_ERR_INVALID, "matrix too large");
  if (bias && bias_dtype != TX_DTYPE_F16 && bias_dtype != TX_DTYPE_BF16)
    return fail(TX_ERR_INVALID, "bias must be CUDA FP16 or BF16 [M]");
  if (on_device && reinterpret_cast<uintptr_t>(blocks) % 8 != 0) return fail(TX_ERR_INVALID, "device blocks must be 8-byte aligned");
  DeviceGuard guard(device);
  Handle *h = new (std::nothrow) Handle;
  if (!h) return fail(TX_ERR_HIP, "host allocation failed");
  h->M = (int)rows;
  h->bpr = (int)bpr;
  h->K = (int)bpr * 16;
  h->device = device;
  h->RG = (h->M + tx::kTileRows - 1) / tx::kTileRows;
  h->Mp = h->RG * tx::kTileRows;
  h->CG = (h->bpr + tx::kTileBlocks - 1) / tx::kTileBlocks;
  h->bp = h->CG * tx::kTileBlocks;
  h->cus = device_cus(device);
  h->gemv_splits = choose_splits(h->RG, h->CG, h->cus);
  const size_t tile_bytes = (size_t)h->RG * h->CG * tx::kTileBytes;

  auto cleanup = [&](hipError_t e) {
    delete h;
    return fail(TX_ERR_HIP, std::string("HIP: ") + hipGetErrorString(e));
  };
  hipError_t e;
  if ((e = hipMalloc(&h->tiles, tile_bytes)) != hipSuccess) return cleanup(e);
  if ((e = hipMalloc(&h->scales, (size_t)h->Mp * sizeof(float))) != hipSuccess) return cleanup(e);
  if (on_device) {
    if ((e = tx::launch_repack(blocks, h->M, h->bpr, h->RG, h->CG, h->tiles, nullptr)) != hipSuccess) return cleanup(e);
    if ((e = hipMemset(h->scales, 0, (size_t)h->Mp * sizeof(float))) != hipSuccess) return cleanup(e);
    if ((e = hipMemcpy(h->scales, scales, (size_t)h->M * sizeof(float), hipMemcpyDeviceToDevice)) != hipSuccess)
      return cleanup(e);
  } else {
    std::vector<uint32_t> host(tile_bytes / 4);
    const int workers = (int)std::max(1u, std::min(16u, std::thread::hardware_concurrency()));
    const int per = (h->RG + workers - 1) / workers;
    std::vector<std::thread> threads;
    for (int w = 0; w < workers; ++w) {
      const int gb = w * per, ge = std::min(h->RG, gb + per);
      if (gb >= ge) break;
      threads.emplace_back(repack_rows, blocks, std::cref(*h), host.data(), gb, ge);
    }
    for (auto &t : threads) t.join();
    std::vector<float> padded_scales(h->Mp, 0.0f);
    std::memcpy(padded_scales.data(), scales, (size_t)h->M * sizeof(float));
    if ((e = hipMemcpy(h->tiles, host.data(), tile_bytes, hipMemcpyHostToDevice)) != hipSuccess) return cleanup(e);
    if ((e = hipMemcpy(h->scales, padded_scales.data(), (size_t)h->Mp * sizeof(float), hipMemcpyHostToDevice)) != hipSuccess)
      return cleanup(e);
  }
  if (bias) {
    if ((e = hipMalloc(&h->bias, (size_t)h->M * 2)) != hipSuccess) return cleanup(e);
    if ((e = hipMemcpy(h->bias, bias, (size_t)h->M * 2, hipMemcpyDeviceToDevice)) != hipSuccess) return cleanup(e);
    h->bias_dtype = bias_dtype;
  }
  // Split-K partials of single-token calls; also the output of tx_linear_split when ks == 1.
  if ((e = hipMalloc(&h->partials, (size_t)h->gemv_splits * h->Mp * sizeof(float))) != hipSuccess) return cleanup(e);
  if ((e = hipDeviceSynchronize()) != hipSuccess) return cleanup(e);
  *handle_out = reinterpret_cast<uint64_t>(h);
  return TX_OK;
}

// ---- Static scratch of tx_linear_noalloc (the array itself is defined above the namespace) ----
constexpr int kMaxScratchDevices = 64;
std::mutex g_scratch_mutex;
float *g_scratch_address[kMaxScratchDevices] = {};

// Device address of `scratch` on `device`, which must be current; looked up once per device.
int scratch_address(int device, float **out) {
  if (device < 0 || device >= kMaxScratchDevices) return fail(TX_ERR_INVALID, "linear_noalloc: device ordinal out of range");
  std::lock_guard<std::mutex> lock(g_scratch_mutex);
  if (!g_scratch_address[device]) {
    void *address = nullptr;
    const hipError_t e = hipGetSymbolAddress(&address, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !address)
      return fail(TX_ERR_HIP, std::string("linear_noalloc: hipGetSymbolAddress(scratch): ") + hipGetErrorString(e));
    g_scratch_address[device] = static_cast<float *>(address);
  }
  *out = g_scratch_address[device];
  return TX_OK;
}

// Bytes the workgroups of a one-token GEMV of `h` read in all to normalize their x themselves (each
// reads the whole residual, every split of the producer's partials, its bias and the weight), up to
// which tx_linear_split_norm and tx_linear_swiglu_norm run.
constexpr int64_t kNormReadBudget = 64ll << 20;

// GemvParams::norm_* for tx_linear_split_norm and tx_linear_swiglu_norm (`workgroups`: the GEMV's);
// TX_OK, or the failure status with nothing launched.
int set_norm_source(tx::GemvParams &p, const Handle *h, const Handle *d, const float *residual_in, float *residual_out,
                    const void *weight, float eps, int64_t workgroups, const char *who) {
  if (!d) return fail(TX_ERR_INVALID, std::string(who) + ": null delta handle");
  if (!residual_in || !residual_out || !weight) return fail(TX_ERR_INVALID, std::string(who) + ": null pointer");
  if (residual_in == residual_out)
    return fail(TX_ERR_INVALID, std::string(who) + ": the updated residual needs its own buffer (the GEMV's "
                                                   "workgroups read residual_in while one writes residual_out)");
  if (reinterpret_cast<uintptr_t>(residual_in) % 16 || reinterpret_cast<uintptr_t>(residual_out) % 16 ||
      reinterpret_cast<uintptr_t>(weight) % 16)
    return fail(TX_ERR_INVALID, std::string(who) + ": residuals and weight must be 16-byte aligned");
  if (d->M != h->K) return fail(TX_ERR_INVALID, std::string(who) + ": the delta handle's output size must equal K");
  if (d->device != h->device) return fail(TX_ERR_INVALID, std::string(who) + ": handles on different devices");
  if (d->bias && d->bias_dtype != TX_DTYPE_BF16) return fail(TX_ERR_INVALID, std::string(who) + ": the delta bias must be BF16");
  const int64_t reads = workgroups * (int64_t)h->K * (4 * (d->gemv_splits + 1) + 4);
  if (h->lut || h->K > tx::kNormMaxHidden || d->gemv_splits > tx::kNormMaxSplits || reads > kNormReadBudget)
    return fail(TX_ERR_UNSUPPORTED, std::string(who) + ": the normalization does not fit the GEMV (LUT handle, "
                                                       "K above 2048, more than 8 delta splits, or too many "
                                                       "workgroups reading the whole row); use "
                                                       "tx_add_rmsnorm_split and the plain call");
  p.norm_h = residual_in;
  p.norm_h_out = residual_out;
  p.norm_partials = d->partials;
  p.norm_bias = static_cast<const uint16_t *>(d->bias);
  p.norm_weight = static_cast<const uint16_t *>(weight);
  p.norm_eps = eps;
  p.norm_ks = d->gemv_splits;
  p.norm_Mp = d->Mp;
  return TX_OK;
}
}  // namespace

extern "C" {

const char *tx_last_error(void) { return g_last_error.c_str(); }

int tx_pack_encoded(const uint8_t *blocks, int64_t blocks_bytes, const float *scales, int64_t rows, const void *bias,
                    int bias_dtype, int device, uint64_t *handle_out) {
  return pack_common(blocks, blocks_bytes, scales, rows, bias, bias_dtype, device, false, handle_out);
}

int tx_pack_encoded_device(const uint8_t *blocks, int64_t blocks_bytes, const float *scales, int64_t rows,
                           const void *bias, int bias_dtype, int device, uint64_t *handle_out) {
  return pack_common(blocks, blocks_bytes, scales, rows, bias, bias_dtype, device, true, handle_out);
}

int tx_concat_rows(const uint64_t *handles, int count, uint64_t *handle_out) {
  g_last_error.clear();
  if (!handles || !handle_out || count < 1 || count > 64) return fail(TX_ERR_INVALID, "concat_rows: 1 to 64 handles and an output");
  std::vector<const Handle *> src(count);
  int64_t rows = 0;
  for (int i = 0; i < count; ++i) {
    src[i] = as_handle(handles[i]);
    if (!src[i]) return fail(TX_ERR_INVALID, "concat_rows: null Texelator handle");
    const Handle &a = *src[i], &first = *src[0];
    if (a.K != first.K || a.device != first.device)
      return fail(TX_ERR_INVALID, "concat_rows: the handles must share K and the device");
    if (i + 1 < count && a.M % tx::kTileRows != 0)
      return fail(TX_ERR_INVALID, "concat_rows: every handle but the last needs a multiple of 16 rows");
    if ((a.bias != nullptr) != (first.bias != nullptr) || (a.bias && a.bias_dtype != first.bias_dtype))
      return fail(TX_ERR_INVALID, "concat_rows: all handles or none carry a bias, of one dtype");
    if (a.lut != first.lut) return fail(TX_ERR_INVALID, "concat_rows: the handles use different palette tables");
    rows += a.M;
  }
  if (rows > (1 << 30)) return fail(TX_ERR_INVALID, "matrix too large");
  const Handle &first = *src[0];
  DeviceGuard guard(first.device);
  Handle *h = new (std::nothrow) Handle;
  if (!h) return fail(TX_ERR_HIP, "host allocation failed");
  h->M = (int)rows;
  h->bpr = first.bpr;
  h->K = first.K;
  h->device = first.device;
  h->RG = (h->M + tx::kTileRows - 1) / tx::kTileRows;
  h->Mp = h->RG * tx::kTileRows;
  h->CG = first.CG;
  h->bp = first.bp;
  h->cus = first.cus;
  h->lookahead = first.lookahead;
  h->prefill_threshold = first.prefill_threshold;
  h->prefill_tile_rows = first.prefill_tile_rows;
  h->prefill_backend = first.prefill_backend;
  h->lut = first.lut;
  h->gemv_splits = choose_splits(h->RG, h->CG, h->cus);
  auto cleanup = [&](hipError_t e) {
    delete h;
    return fail(TX_ERR_HIP, std::string("HIP: ") + hipGetErrorString(e));
  };
  hipError_t e;
  if ((e = hipMalloc(&h->tiles, (size_t)h->RG * h->CG * tx::kTileBytes)) != hipSuccess) return cleanup(e);
  if ((e = hipMalloc(&h->scales, (size_t)h->Mp * sizeof(float))) != hipSuccess) return cleanup(e);
  if (first.bias) {
    if ((e = hipMalloc(&h->bias, (size_t)h->M * 2)) != hipSuccess) return cleanup(e);
    h->bias_dtype = first.bias_dtype;
  }
  // Tiles are row-group major, so each source's row groups follow the previous source's; every
  // source but the last fills its row groups, so rows keep their order and the padding stays last.
  int64_t g = 0, row = 0;
  for (const Handle *a : src) {
    const size_t tile_bytes = (size_t)a->RG * a->CG * tx::kTileBytes;
    if ((e = hipMemcpy(reinterpret_cast<char *>(h->tiles) + (size_t)g * h->CG * tx::kTileBytes, a->tiles, tile_bytes,
                       hipMemcpyDeviceToDevice)) != hipSuccess)
      return cleanup(e);
    if ((e = hipMemcpy(h->scales + row, a->scales, (size_t)a->Mp * sizeof(float), hipMemcpyDeviceToDevice)) != hipSuccess)
      return cleanup(e);
    if (a->bias && (e = hipMemcpy(static_cast<char *>(h->bias) + (size_t)row * 2, a->bias, (size_t)a->M * 2,
                                  hipMemcpyDeviceToDevice)) != hipSuccess)
      return cleanup(e);
    g += a->RG;
    row += a->M;
  }
  if ((e = hipMalloc(&h->partials, (size_t)h->gemv_splits * h->Mp * sizeof(float))) != hipSuccess) return cleanup(e);
  if ((e = hipDeviceSynchronize()) != hipSuccess) return cleanup(e);
  *handle_out = reinterpret_cast<uint64_t>(h);
  return TX_OK;
}

int tx_linear(uint64_t value, const void *x, int x_dtype, int64_t x_numel, int64_t x_last, int device, void *y,
              void *workspace, int64_t workspace_bytes, void *stream) {
  g_last_error.clear();
  Handle *h = as_handle(value);
  if (!h) return fail(TX_ERR_INVALID, "null Texelator handle");
  if (x_dtype != TX_DTYPE_BF16 && x_dtype != TX_DTYPE_F16) return fail(TX_ERR_INVALID, "input must be contiguous CUDA FP16 or BF16");
  if (x_last != h->K || device != h->device) return fail(TX_ERR_INVALID, "input shape/device mismatch");
  if (!x || !y) return fail(TX_ERR_INVALID, "null input or output pointer");
  if (reinterpret_cast<uintptr_t>(x) % 16 != 0) return fail(TX_ERR_INVALID, "input must be 16-byte aligned");
  const bool f16 = x_dtype == TX_DTYPE_F16;
  const int64_t tokens = x_numel / h->K;
  if (tokens <= 0) return TX_OK;
  DeviceGuard guard(h->device);
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  if (tokens >= h->prefill_threshold && tokens > 1) {
    if (h->bias && h->bias_dtype != x_dtype)
      return fail(TX_ERR_INVALID, f16 ? "FP16 prefill requires an FP16 bias" : "BF16 prefill requires a BF16 bias");
    return run_prefill(h, prefill_choice(h, tokens), x, f16, tokens, y, workspace, workspace_bytes, s);
  }
  if (h->bias && h->bias_dtype != x_dtype) return fail(TX_ERR_INVALID, "input and bias dtypes must match");
  // A caller workspace large enough for the one-token split-K partials keeps concurrent calls on
  // one handle apart; without one the handle's own buffer is used (calls must then not overlap).
  const int64_t need = gemv_partials_bytes(h, tokens);
  const bool own = need > 0 && workspace && workspace_bytes >= need && reinterpret_cast<uintptr_t>(workspace) % 16 == 0;
  return run_gemv(h, x, f16, tokens, y, false, s, own ? static_cast<float *>(workspace) : h->partials);
}

int tx_linear_add_bias(uint64_t value, const void *x, const void *bias, void *y, void *stream) {
  g_last_error.clear();
  Handle *h = as_handle(value);
  if (!h) return fail(TX_ERR_INVALID, "null Texelator handle");
  if (!x || !bias || !y) return fail(TX_ERR_INVALID, "null input, bias or output pointer");
  if (reinterpret_cast<uintptr_t>(x) % 16 != 0) return fail(TX_ERR_INVALID, "input must be 16-byte aligned");
  if (reinterpret_cast<uintptr_t>(bias) % 2 != 0) return fail(TX_ERR_INVALID, "bias must be 2-byte aligned");
  if (h->bias) return fail(TX_ERR_INVALID, "linear_add_bias: the handle carries its own bias");
  DeviceGuard guard(h->device);
  tx::GemvParams p{};
  p.lut = h->lut;
  p.tiles = h->tiles;
  p.scales = h->scales;
  p.x = x;
  p.bias = bias;
  p.bias_round_first = 1;
  p.y = y;
  p.M = h->M;
  p.K = h->K;
  p.Mp = h->Mp;
  p.RG = h->RG;
  p.CG = h->CG;
  p.tokens = 1;
  p.ks = h->gemv_splits;
  p.partials = h->partials;
  p.fused = one_token_fused(h) ? 1 : 0;
  TX_HIP(tx::launch_gemv(p, h->lookahead, false, reinterpret_cast<hipStream_t>(stream)));
  return TX_OK;
}

int tx_linear_noalloc(uint64_t value, const void *x, int x_dtype, int64_t x_numel, int64_t x_last, int device, void *y,
                      void *stream) {
  g_last_error.clear();
  Handle *h = as_handle(value);
  if (!h) return fail(TX_ERR_INVALID, "null Texelator handle");
  if (x_dtype != TX_DTYPE_BF16 && x_dtype != TX_DTYPE_F16) return fail(TX_ERR_INVALID, "input must be contiguous CUDA FP16 or BF16");
  if (x_last != h->K || device != h->device) return fail(TX_ERR_INVALID, "input shape/device mismatch");
  if (!x || !y) return fail(TX_ERR_INVALID, "null input or output pointer");
  if (reinterpret_cast<uintptr_t>(x) % 16 != 0) return fail(TX_ERR_INVALID, "input must be 16-byte aligned");
  const bool f16 = x_dtype == TX_DTYPE_F16;
  const int64_t tokens = x_numel / h->K;
  if (tokens <= 0) return TX_OK;
  const bool prefill = tokens >= h->prefill_threshold && tokens > 1;
  // The dense-scratch backend runs a library GEMM that creates handles, descriptors and plans on
  // first use: not allocation-free, so this entry point refuses it before launching anything.
  if (prefill && prefill_choice(h, tokens) == kDenseBackend)
    return fail(TX_ERR_UNSUPPORTED, "linear_noalloc: prefill backend 1 (dense scratch + library GEMM) allocates; "
                                    "use tx_linear with a workspace or another prefill backend");
  if (prefill && tokens > (1 << 20)) return fail(TX_ERR_INVALID, "token count exceeds the prefill limit (1048576)");
  if (!prefill && tokens > 65535) return fail(TX_ERR_INVALID, "token grid exceeds the HIP grid.z limit");
  const int64_t need = prefill ? prefill_call_bytes(h, tokens) : gemv_partials_bytes(h, tokens);
  if (need > (int64_t)kScratchBytes)
    return fail(TX_ERR_INVALID, "linear_noalloc: the call's scratch needs " + std::to_string(need) +
                                    " bytes, more than the 33554432-byte static scratch; use tx_linear with a workspace");
  if (h->bias && h->bias_dtype != x_dtype)
    return fail(TX_ERR_INVALID, prefill ? (f16 ? "FP16 prefill requires an FP16 bias" : "BF16 prefill requires a BF16 bias")
                                        : "input and bias dtypes must match");
  DeviceGuard guard(h->device);
  float *partials = nullptr;
  if (const int status = scratch_address(h->device, &partials)) return status;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  if (prefill) return run_prefill(h, prefill_choice(h, tokens), x, f16, tokens, y, partials, (int64_t)kScratchBytes, s);
  return run_gemv(h, x, f16, tokens, y, false, s, partials);
}

int tx_quantize_activation_fp4(const void *x, int x_dtype, int64_t tokens, int64_t K, uint8_t *packed, uint8_t *scales,
                               int device, void *stream) {
  g_last_error.clear();
  if (x_dtype != TX_DTYPE_BF16) return fail(TX_ERR_INVALID, "activation must be contiguous CUDA BF16 [tokens,K]");
  if (K <= 0 || K % 32 != 0) return fail(TX_ERR_INVALID, "activation K must be a positive multiple of 32");
  if (tokens < 0 || tokens * (K / 32) > 0x7FFFFFFF) return fail(TX_ERR_INVALID, "activation too large");
  if (!x || !packed || !scales) return fail(TX_ERR_INVALID, "null pointer");
  if (reinterpret_cast<uintptr_t>(x) % 16 != 0 || reinterpret_cast<uintptr_t>(packed) % 16 != 0)
    return fail(TX_ERR_INVALID, "activation and packed output must be 16-byte aligned");
  if (tokens == 0) return TX_OK;
  DeviceGuard guard(device);
  TX_HIP(tx::launch_quantize_activation_fp4(static_cast<const uint16_t *>(x), tokens, (int)K, packed, scales,
                                            reinterpret_cast<hipStream_t>(stream)));
  return TX_OK;
}

int tx_decode_weight_fp4(uint64_t value, uint8_t *packed, uint8_t *scales, void *stream) {
  g_last_error.clear();
  Handle *h = as_handle(value);
  if (!h) return fail(TX_ERR_INVALID, "null Texelator handle");
  if (h->K % 32 != 0) return fail(TX_ERR_INVALID, "weight K must be a multiple of 32");
  if (!packed || !scales) return fail(TX_ERR_INVALID, "null pointer");
  if (reinterpret_cast<uintptr_t>(packed) % 16 != 0) return fail(TX_ERR_INVALID, "packed output must be 16-byte aligned");
  DeviceGuard guard(h->device);
  TX_HIP(tx::launch_quantize_weight_fp4(h->tiles, h->scales, h->lut, h->M, h->K, h->RG, h->CG, packed, scales,
                                        reinterpret_cast<hipStream_t>(stream)));
  return TX_OK;
}

int tx_fp4_gemm(const uint8_t *x_packed, const uint8_t *x_scales, const uint8_t *w_packed, const uint8_t *w_scales,
                const void *bias, int64_t tokens, int64_t M, int64_t K, void *y, int device, void *stream) {
  g_last_error.clear();
  if (K <= 0 || K % 64 != 0) return fail(TX_ERR_INVALID, "FP4 GEMM K must be a positive multiple of 64");
  if (M <= 0 || M > 0x7FFFFFFF || tokens < 0 || tokens > 0x7FFFFFFF) return fail(TX_ERR_INVALID, "FP4 GEMM shape out of range");
  if (!x_packed || !x_scales || !w_packed || !w_scales || !y) return fail(TX_ERR_INVALID, "null pointer");
  if (reinterpret_cast<uintptr_t>(x_packed) % 16 != 0 || reinterpret_cast<uintptr_t>(w_packed) % 16 != 0)
    return fail(TX_ERR_INVALID, "packed operands must be 16-byte aligned");
  if (tokens == 0) return TX_OK;
  DeviceGuard guard(device);
  TX_HIP(tx::launch_fp4_gemm(x_packed, x_scales, w_packed, w_scales, static_cast<const uint16_t *>(bias),
                             static_cast<uint16_t *>(y), (int)tokens, (int)M, (int)K,
                             reinterpret_cast<hipStream_t>(stream)));
  return TX_OK;
}

int tx_noalloc_scratch_bytes(int64_t *bytes) {
  g_last_error.clear();
  if (!bytes) return fail(TX_ERR_INVALID, "null output");
  *bytes = (int64_t)kScratchBytes;
  return TX_OK;
}

int tx_linear_f32(uint64_t value, const void *x, int64_t tokens, float *y, void *stream) {
  g_last_error.clear();
  Handle *h = as_handle(value);
  if (!h) return fail(TX_ERR_INVALID, "null Texelator handle");
  if (!x || !y) return fail(TX_ERR_INVALID, "null input or output pointer");
  if (reinterpret_cast<uintptr_t>(x) % 16 != 0) return fail(TX_ERR_INVALID, "input must be 16-byte aligned");
  if (tokens <= 0) return TX_OK;
  DeviceGuard guard(h->device);
  return run_gemv(h, x, false, tokens, y, true, reinterpret_cast<hipStream_t>(stream), h->partials);
}

int tx_prefill(uint64_t value, int candidate, const void *x, int x_dtype, int64_t tokens, void *y, void *workspace,
               int64_t workspace_bytes, void *stream) {
  g_last_error.clear();
  Handle *h = as_handle(value);
  if (!h) return fail(TX_ERR_INVALID, "null Texelator handle");
  if (!x || !y) return fail(TX_ERR_INVALID, "null input or output pointer");
  if (x_dtype != TX_DTYPE_BF16 && x_dtype != TX_DTYPE_F16) return fail(TX_ERR_INVALID, "input must be FP16 or BF16");
  if (reinterpret_cast<uintptr_t>(x) % 16 != 0) return fail(TX_ERR_INVALID, "input must be 16-byte aligned");
  if (!tx::prefill_candidate_eligible(candidate, h->M, h->K)) return fail(TX_ERR_INVALID, "unknown or ineligible prefill candidate");
  const bool f16 = x_dtype == TX_DTYPE_F16;
  if (h->bias && h->bias_dtype != x_dtype)
    return fail(TX_ERR_INVALID, f16 ? "FP16 prefill requires an FP16 bias" : "BF16 prefill requires a BF16 bias");
  if (tokens <= 0) return TX_OK;
  DeviceGuard guard(h->device);
  return run_prefill(h, candidate, x, f16, tokens, y, workspace, workspace_bytes, reinterpret_cast<hipStream_t>(stream));
}

int tx_workspace_bytes(uint64_t value, int64_t tokens, int64_t *bytes) {
  g_last_error.clear();
  Handle *h = as_handle(value);
  if (!h) return fail(TX_ERR_INVALID, "null Texelator handle");
  if (!bytes) return fail(TX_ERR_INVALID, "null output");
  if (tokens > 1 && tokens >= h->prefill_threshold) *bytes = prefill_call_bytes(h, tokens);
  else *bytes = tokens > 1 ? prefill_workspace_bytes(h, tokens) : gemv_partials_bytes(h, tokens);
  return TX_OK;
}

int tx_set_lookahead(uint64_t value, int lookahead) {
  g_last_error.clear();
  Handle *h = as_handle(value);
  if (!h) return fail(TX_ERR_INVALID, "null Texelator handle");
  if (!tx::gemv_lookahead_supported(lookahead)) return fail(TX_ERR_INVALID, "lookahead must be one of 1,2,3,4,6,8");
  h->lookahead = lookahead;
  return TX_OK;
}

int tx_set_prefill(uint64_t value, int threshold, int tile_rows) {
  g_last_error.clear();
  Handle *h = as_handle(value);
  if (!h) return fail(TX_ERR_INVALID, "null Texelator handle");
  if (threshold < 1) return fail(TX_ERR_INVALID, "prefill threshold must be positive");
  if (tile_rows < 16 || tile_rows % 16 != 0) return fail(TX_ERR_INVALID, "prefill tile rows must be a positive multiple of 16");
  h->prefill_threshold = threshold;
  h->prefill_tile_rows = tile_rows;
  return TX_OK;
}

int tx_set_palette_table(uint64_t value, const float *device_table) {
  g_last_error.clear();
  Handle *h = as_handle(value);
  if (!h) return fail(TX_ERR_INVALID, "null Texelator handle");
  if (device_table && reinterpret_cast<uintptr_t>(device_table) % 16 != 0)
    return fail(TX_ERR_INVALID, "palette table must be 16-byte aligned");
  h->lut = reinterpret_cast<const float4 *>(device_table);
  return TX_OK;
}

int tx_set_prefill_backend(uint64_t value, int backend) {
  g_last_error.clear();
  Handle *h = as_handle(value);
  if (!h) return fail(TX_ERR_INVALID, "null Texelator handle");
  if (backend < 0 || backend > tx::kPrefillLast) {
    std::string message = "prefill backend must be 0 or 2-4 (default tile), 1 (dense scratch and hipBLASLt)";
    for (int c = tx::kPrefillFirst; c <= tx::kPrefillLast; ++c)
      message += std::string(c == tx::kPrefillLast ? ", or " : ", ") + std::to_string(c) + " (" +
                 tx::prefill_candidate_name(c) + ")";
    return fail(TX_ERR_INVALID, message);
  }
  h->prefill_backend = backend;
  return TX_OK;
}

int tx_handle_info(uint64_t value, int64_t *out, int n) {
  g_last_error.clear();
  Handle *h = as_handle(value);
  if (!h) return fail(TX_ERR_INVALID, "null Texelator handle");
  if (!out || n < 0) return fail(TX_ERR_INVALID, "invalid output buffer");
  const int64_t info[11] = {h->M, h->K, h->prefill_threshold, h->prefill_tile_rows, h->prefill_backend, 0, 0,
                            h->lookahead, h->device, h->gemv_splits, h->lut != nullptr};
  for (int i = 0; i < n && i < 11; ++i) out[i] = info[i];
  return TX_OK;
}

int tx_free(uint64_t value) {
  g_last_error.clear();
  Handle *h = as_handle(value);
  if (!h) return fail(TX_ERR_INVALID, "null Texelator handle");
  delete h;
  return TX_OK;
}

int tx_palette_probe(float *host_out) {
  g_last_error.clear();
  if (!host_out) return fail(TX_ERR_INVALID, "null output");
  float *device_out = nullptr;
  const size_t bytes = (size_t)255 * 255 * 8 * sizeof(float);
  TX_HIP(hipMalloc(&device_out, bytes));
  hipError_t e = tx::launch_palette_probe(device_out, nullptr);
  if (e == hipSuccess) e = hipMemcpy(host_out, device_out, bytes, hipMemcpyDeviceToHost);
  (void)hipFree(device_out);
  if (e != hipSuccess) return fail(TX_ERR_HIP, std::string("HIP: ") + hipGetErrorString(e));
  return TX_OK;
}

int tx_decode_dense(uint64_t value, int dtype, uint16_t *out, void *stream) {
  g_last_error.clear();
  Handle *h = as_handle(value);
  if (!h) return fail(TX_ERR_INVALID, "null Texelator handle");
  if (!out) return fail(TX_ERR_INVALID, "null output");
  if (dtype != TX_DTYPE_BF16 && dtype != TX_DTYPE_F16) return fail(TX_ERR_INVALID, "decode_dense: dtype must be FP16 or BF16");
  DeviceGuard guard(h->device);
  TX_HIP(tx::launch_decode_dense(h->tiles, h->scales, h->lut, h->M, h->K, h->RG, h->CG, dtype == TX_DTYPE_F16, out,
                                 reinterpret_cast<hipStream_t>(stream)));
  return TX_OK;
}

int tx_stream_read(const void *data, int64_t bytes, uint32_t *sink, void *stream) {
  g_last_error.clear();
  if (!data || !sink) return fail(TX_ERR_INVALID, "null data or sink");
  if (bytes <= 0 || bytes % 16 != 0 || reinterpret_cast<uintptr_t>(data) % 16 != 0)
    return fail(TX_ERR_INVALID, "stream_read: bytes must be a positive multiple of 16 and data 16-byte aligned");
  TX_HIP(tx::launch_stream_read(data, (size_t)bytes, sink, reinterpret_cast<hipStream_t>(stream)));
  return TX_OK;
}

int tx_kernel_info(int candidate, int64_t *out, int n) {
  g_last_error.clear();
  if (!out || n < 0) return fail(TX_ERR_INVALID, "invalid output buffer");
  hipFuncAttributes attr{};
  int lds = 0, bt = 0, bn = 0, bk = 0, resident = 0;
  if (candidate >= 100) {
    if (!tx::gemv_lookahead_supported(candidate - 100)) return fail(TX_ERR_INVALID, "unknown kernel candidate");
    TX_HIP(tx::gemv_kernel_attributes(candidate - 100, &attr));
    bt = 1;
    bn = tx::kTileRows;
    bk = tx::kTileK;
    // Occupancy for the 27B-class K of 5120 (40 tile columns of staged x).
    lds = 40 * tx::kTileK * 2;
    resident = tx::gemv_resident_per_cu(candidate - 100, 40);
  } else {
    if (!tx::prefill_candidate_name(candidate)) return fail(TX_ERR_INVALID, "unknown kernel candidate");
    TX_HIP(tx::prefill_kernel_attributes(candidate, &attr, &lds));
    tx::prefill_candidate_shape(candidate, &bt, &bn, &bk);
    resident = tx::prefill_resident_per_cu(candidate);
  }
  const int64_t info[9] = {attr.numRegs, (int64_t)attr.sharedSizeBytes, (int64_t)attr.localSizeBytes,
                           attr.maxThreadsPerBlock, lds, bt, bn, bk, resident};
  for (int i = 0; i < n && i < 9; ++i) out[i] = info[i];
  return TX_OK;
}

const char *tx_candidate_name(int candidate) { return tx::prefill_candidate_name(candidate); }

int tx_add_rmsnorm(float *residual, const void *delta, const void *weight, float eps, void *out, int64_t rows,
                   int64_t hidden, void *stream) {
  g_last_error.clear();
  if (!residual || !weight || !out || rows < 0 || hidden <= 0 || hidden > (1 << 24) || hidden % 4)
    return fail(TX_ERR_INVALID, "add_rmsnorm: invalid arguments (hidden must be a positive multiple of 4)");
  if (rows == 0) return TX_OK;
  TX_HIP(tx::launch_add_rmsnorm(residual, static_cast<const uint16_t *>(delta), static_cast<const uint16_t *>(weight),
                                eps, static_cast<uint16_t *>(out), rows, (int)hidden, reinterpret_cast<hipStream_t>(stream)));
  return TX_OK;
}

int tx_add_rmsnorm_bf16(const void *residual, const void *delta, const void *weight, float eps, void *sum_out, void *out,
                        int64_t rows, int64_t hidden, void *stream) {
  g_last_error.clear();
  if (!residual || !weight || !out || (delta && !sum_out) || rows < 0 || rows > 0x7FFFFFFF || hidden <= 0 ||
      hidden > (1 << 24) || hidden % 4)
    return fail(TX_ERR_INVALID, "add_rmsnorm_bf16: invalid arguments (hidden must be a positive multiple of 4; "
                                "a delta needs sum_out)");
  for (const void *ptr : {residual, delta, weight, static_cast<const void *>(sum_out), static_cast<const void *>(out)})
    if (reinterpret_cast<uintptr_t>(ptr) % 8) return fail(TX_ERR_INVALID, "add_rmsnorm_bf16: pointers must be 8-byte aligned");
  if (rows == 0) return TX_OK;
  TX_HIP(tx::launch_add_rmsnorm_bf16(static_cast<const uint16_t *>(residual), static_cast<const uint16_t *>(delta),
                                     static_cast<const uint16_t *>(weight), eps, delta ? static_cast<uint16_t *>(sum_out) : nullptr,
                                     static_cast<uint16_t *>(out), rows, (int)hidden, reinterpret_cast<hipStream_t>(stream)));
  return TX_OK;
}

int tx_linear_split(uint64_t value, const void *x, void *stream) {
  g_last_error.clear();
  Handle *h = as_handle(value);
  if (!h) return fail(TX_ERR_INVALID, "null Texelator handle");
  if (!x) return fail(TX_ERR_INVALID, "null input pointer");
  if (reinterpret_cast<uintptr_t>(x) % 16 != 0) return fail(TX_ERR_INVALID, "input must be 16-byte aligned");
  if (h->bias && h->bias_dtype != TX_DTYPE_BF16) return fail(TX_ERR_INVALID, "linear_split: the bias must be BF16");
  DeviceGuard guard(h->device);
  return run_gemv_split(h, x, reinterpret_cast<hipStream_t>(stream));
}

int tx_linear_swiglu(uint64_t value, const void *x, void *out, void *stream) {
  g_last_error.clear();
  Handle *h = as_handle(value);
  if (!h) return fail(TX_ERR_INVALID, "null Texelator handle");
  if (!x || !out) return fail(TX_ERR_INVALID, "null input or output pointer");
  if (reinterpret_cast<uintptr_t>(x) % 16 != 0) return fail(TX_ERR_INVALID, "input must be 16-byte aligned");
  if (h->M % 32 != 0) return fail(TX_ERR_INVALID, "linear_swiglu: the handle must hold [gate | up] with 16-row aligned halves");
  if (h->gemv_splits != 1 || h->CG > tx::kGemvMaxLdsColumns || h->lut)
    return fail(TX_ERR_UNSUPPORTED, "linear_swiglu: needs a one-split, non-LUT handle with K <= 16384");
  if (h->bias && h->bias_dtype != TX_DTYPE_BF16) return fail(TX_ERR_INVALID, "linear_swiglu: the bias must be BF16");
  DeviceGuard guard(h->device);
  tx::GemvParams p{};
  p.tiles = h->tiles;
  p.scales = h->scales;
  p.x = x;
  p.bias = h->bias;
  p.y = out;
  p.M = h->M;
  p.K = h->K;
  p.Mp = h->Mp;
  p.RG = h->RG;
  p.CG = h->CG;
  p.ks = 1;
  p.tokens = 1;
  TX_HIP(tx::launch_gemv_swiglu(p, h->lookahead, reinterpret_cast<hipStream_t>(stream)));
  return TX_OK;
}

int tx_linear_swiglu_pair(uint64_t gate, uint64_t up, const void *x, void *out, void *stream) {
  g_last_error.clear();
  Handle *hg = as_handle(gate);
  Handle *hu = as_handle(up);
  if (!hg || !hu) return fail(TX_ERR_INVALID, "null Texelator handle");
  if (!x || !out) return fail(TX_ERR_INVALID, "null input or output pointer");
  if (reinterpret_cast<uintptr_t>(x) % 16 != 0) return fail(TX_ERR_INVALID, "input must be 16-byte aligned");
  if (hg->M != hu->M || hg->K != hu->K || hg->device != hu->device)
    return fail(TX_ERR_INVALID, "linear_swiglu_pair: gate and up must have the same shape and device");
  if (hg->CG > tx::kGemvMaxLdsColumns || hg->lut || hu->lut || hg->bias || hu->bias)
    return fail(TX_ERR_UNSUPPORTED, "linear_swiglu_pair: needs non-LUT handles without a bias, K <= 16384");
  DeviceGuard guard(hg->device);
  tx::GemvParams p{};
  p.tiles = hg->tiles;
  p.scales = hg->scales;
  p.tiles_up = hu->tiles;
  p.scales_up = hu->scales;
  p.x = x;
  p.y = out;
  p.M = 2 * hg->M;
  p.K = hg->K;
  p.Mp = hg->Mp;
  p.RG = hg->RG;
  p.CG = hg->CG;
  p.ks = 1;
  p.tokens = 1;
  TX_HIP(tx::launch_gemv_swiglu(p, hg->lookahead, reinterpret_cast<hipStream_t>(stream)));
  return TX_OK;
}

int tx_linear_swiglu_prefill(uint64_t value, const void *x, int64_t tokens, void *out, void *stream) {
  g_last_error.clear();
  Handle *h = as_handle(value);
  if (!h) return fail(TX_ERR_INVALID, "null Texelator handle");
  if (!x || !out) return fail(TX_ERR_INVALID, "null input or output pointer");
  if (reinterpret_cast<uintptr_t>(x) % 16 != 0) return fail(TX_ERR_INVALID, "input must be 16-byte aligned");
  if (h->M % 32 != 0) return fail(TX_ERR_INVALID, "linear_swiglu_prefill: the handle must hold [gate | up] with 16-row aligned halves");
  if (h->bias && h->bias_dtype != TX_DTYPE_BF16) return fail(TX_ERR_INVALID, "linear_swiglu_prefill: the bias must be BF16");
  if (tokens > (1 << 20)) return fail(TX_ERR_INVALID, "token count exceeds the prefill limit (1048576)");
  if (tokens < 2 || tokens < h->prefill_threshold)
    return fail(TX_ERR_UNSUPPORTED, "linear_swiglu_prefill: the call is below the prefill threshold (use tx_linear_swiglu "
                                    "for one token, tx_linear + tx_swiglu otherwise)");
  const int candidate = prefill_choice(h, tokens);
  if (!tx::prefill_swiglu_supported(candidate) || tx::prefill_splits(h->M, h->CG, tokens, h->cus) != 1)
    return fail(TX_ERR_UNSUPPORTED, "linear_swiglu_prefill: this call's prefill runs the pair tile or the dense "
                                    "backend, or splits K (use tx_linear + tx_swiglu)");
  DeviceGuard guard(h->device);
  tx::PrefillParams p{};
  p.lut = h->lut;
  p.tiles = h->tiles;
  p.scales = h->scales;
  p.x = x;
  p.bias = h->bias;
  p.y = out;
  p.M = h->M;
  p.K = h->K;
  p.Mp = h->Mp;
  p.RG = h->RG;
  p.CG = h->CG;
  p.tokens = (int)tokens;
  p.ks = 1;
  TX_HIP(tx::launch_prefill_swiglu(p, candidate, reinterpret_cast<hipStream_t>(stream)));
  return TX_OK;
}

// The prefill-sized K-split partials of a handle for `tokens` tokens in a caller's buffer
// (tx_prefill_split), as the prefill reduce sums and rounds them.
tx::SplitSource prefill_split_source(const Handle *h, const void *partials, int64_t tokens) {
  return tx::SplitSource{static_cast<const float *>(partials), static_cast<const uint16_t *>(h->bias),
                         tx::prefill_splits(h->M, h->CG, tokens, h->cus), h->Mp, (int)tokens, 1};
}

int tx_prefill_split(uint64_t value, const void *x, int64_t tokens, void *workspace, int64_t workspace_bytes,
                     int *splits_out, void *stream) {
  g_last_error.clear();
  Handle *h = as_handle(value);
  if (!h) return fail(TX_ERR_INVALID, "null Texelator handle");
  if (!x || !splits_out) return fail(TX_ERR_INVALID, "prefill_split: null input or splits pointer");
  if (reinterpret_cast<uintptr_t>(x) % 16 != 0) return fail(TX_ERR_INVALID, "input must be 16-byte aligned");
  if (h->bias && h->bias_dtype != TX_DTYPE_BF16) return fail(TX_ERR_INVALID, "prefill_split: the bias must be BF16");
  if (tokens > (1 << 20)) return fail(TX_ERR_INVALID, "token count exceeds the prefill limit (1048576)");
  if (tokens < 2 || tokens < h->prefill_threshold)
    return fail(TX_ERR_UNSUPPORTED, "prefill_split: the call is below the prefill threshold (tx_linear runs the GEMV)");
  const int candidate = prefill_choice(h, tokens);
  if (candidate == kDenseBackend) return fail(TX_ERR_UNSUPPORTED, "prefill_split: the dense backend has no K splits");
  const int ks = tx::prefill_splits(h->M, h->CG, tokens, h->cus);
  if (ks == 1) return fail(TX_ERR_UNSUPPORTED, "prefill_split: this call does not split K (use tx_linear)");
  if (!workspace || workspace_bytes < prefill_workspace_bytes(h, tokens) || reinterpret_cast<uintptr_t>(workspace) % 16 != 0)
    return fail(TX_ERR_INVALID, "prefill_split: workspace missing or too small (see tx_workspace_bytes)");
  DeviceGuard guard(h->device);
  tx::PrefillParams p{};
  p.lut = h->lut;
  p.tiles = h->tiles;
  p.scales = h->scales;
  p.x = x;
  p.bias = h->bias;
  p.M = h->M;
  p.K = h->K;
  p.Mp = h->Mp;
  p.RG = h->RG;
  p.CG = h->CG;
  p.tokens = (int)tokens;
  p.ks = ks;
  p.partials = static_cast<float *>(workspace);
  p.no_reduce = 1;
  TX_HIP(tx::launch_prefill(p, candidate, reinterpret_cast<hipStream_t>(stream)));
  *splits_out = ks;
  return TX_OK;
}

int tx_add_rmsnorm_prefill_split(float *residual, uint64_t delta_handle, const void *partials, int64_t tokens,
                                 const void *weight, float eps, void *out, int64_t hidden, void *stream) {
  g_last_error.clear();
  Handle *h = as_handle(delta_handle);
  if (!h) return fail(TX_ERR_INVALID, "null Texelator handle");
  if (!residual || !partials || !weight || !out || hidden <= 0 || hidden > (1 << 24) || hidden % 4 || tokens < 2 ||
      tokens > (1 << 20))
    return fail(TX_ERR_INVALID, "add_rmsnorm_prefill_split: invalid arguments (hidden a positive multiple of 4, 2..1048576 tokens)");
  if (h->M != hidden) return fail(TX_ERR_INVALID, "add_rmsnorm_prefill_split: the handle's output size must equal hidden");
  if (h->bias && h->bias_dtype != TX_DTYPE_BF16) return fail(TX_ERR_INVALID, "add_rmsnorm_prefill_split: the bias must be BF16");
  DeviceGuard guard(h->device);
  TX_HIP(tx::launch_add_rmsnorm_split(residual, prefill_split_source(h, partials, tokens), static_cast<const uint16_t *>(weight),
                                      eps, static_cast<uint16_t *>(out), tokens, (int)hidden,
                                      reinterpret_cast<hipStream_t>(stream)));
  return TX_OK;
}

int tx_rope_kv_cache_prefill_split(uint64_t qkv_handle, const void *partials, int64_t tokens, const int64_t *positions,
                                   const float *cos_table, const float *sin_table, int heads, int kv_heads, int head_dim,
                                   void *q_out, void *k_cache, void *v_cache, int64_t max_context, void *stream) {
  g_last_error.clear();
  Handle *h = as_handle(qkv_handle);
  if (!h) return fail(TX_ERR_INVALID, "null Texelator handle");
  if (!partials || !positions || !cos_table || !sin_table || !q_out || !k_cache || !v_cache)
    return fail(TX_ERR_INVALID, "rope_kv_cache_prefill_split: null pointer");
  if (heads <= 0 || kv_heads <= 0 || head_dim <= 0 || head_dim % 2 || head_dim > 1024 || max_context <= 0 || tokens < 2 ||
      tokens > 65535 || (int64_t)h->M < (int64_t)(heads + 2 * kv_heads) * head_dim)
    return fail(TX_ERR_INVALID, "rope_kv_cache_prefill_split: invalid shape");
  if (h->bias && h->bias_dtype != TX_DTYPE_BF16) return fail(TX_ERR_INVALID, "rope_kv_cache_prefill_split: the bias must be BF16");
  DeviceGuard guard(h->device);
  TX_HIP(tx::launch_rope_cache_split(prefill_split_source(h, partials, tokens), tokens, positions, cos_table, sin_table,
                                     heads, kv_heads, head_dim, static_cast<uint16_t *>(q_out),
                                     static_cast<uint16_t *>(k_cache), static_cast<uint16_t *>(v_cache), max_context,
                                     reinterpret_cast<hipStream_t>(stream)));
  return TX_OK;
}

int tx_add_rmsnorm_split(float *residual, uint64_t delta_handle, const void *weight, float eps, void *out, int64_t hidden,
                         void *stream) {
  g_last_error.clear();
  Handle *h = as_handle(delta_handle);
  if (!h) return fail(TX_ERR_INVALID, "null Texelator handle");
  if (!residual || !weight || !out || hidden <= 0 || hidden > (1 << 24) || hidden % 4)
    return fail(TX_ERR_INVALID, "add_rmsnorm_split: invalid arguments (hidden must be a positive multiple of 4)");
  if (h->M != hidden) return fail(TX_ERR_INVALID, "add_rmsnorm_split: the handle's output size must equal hidden");
  if (h->bias && h->bias_dtype != TX_DTYPE_BF16) return fail(TX_ERR_INVALID, "add_rmsnorm_split: the bias must be BF16");
  DeviceGuard guard(h->device);
  TX_HIP(tx::launch_add_rmsnorm_split(residual, split_source(h), static_cast<const uint16_t *>(weight), eps,
                                      static_cast<uint16_t *>(out), 1, (int)hidden, reinterpret_cast<hipStream_t>(stream)));
  return TX_OK;
}

int tx_linear_split_norm(uint64_t value, const float *residual_in, float *residual_out, uint64_t delta_handle,
                         const void *weight, float eps, void *stream) {
  g_last_error.clear();
  Handle *h = as_handle(value);
  if (!h) return fail(TX_ERR_INVALID, "null Texelator handle");
  if (h->bias && h->bias_dtype != TX_DTYPE_BF16) return fail(TX_ERR_INVALID, "linear_split_norm: the bias must be BF16");
  tx::GemvParams p{};
  p.tiles = h->tiles;
  p.scales = h->scales;
  p.M = h->M;
  p.K = h->K;
  p.Mp = h->Mp;
  p.RG = h->RG;
  p.CG = h->CG;
  p.tokens = 1;
  p.ks = h->gemv_splits;
  p.partials = h->partials;
  p.force_partials = 1;
  const int status = set_norm_source(p, h, as_handle(delta_handle), residual_in, residual_out, weight, eps,
                                     (int64_t)h->RG * h->gemv_splits, "linear_split_norm");
  if (status != TX_OK) return status;
  DeviceGuard guard(h->device);
  TX_HIP(tx::launch_gemv(p, h->lookahead, true, reinterpret_cast<hipStream_t>(stream)));
  return TX_OK;
}

int tx_linear_split_embed_norm(uint64_t value, const void *embed, int64_t vocab, const int64_t *token,
                               float *residual_out, const void *weight, float eps, void *stream) {
  g_last_error.clear();
  Handle *h = as_handle(value);
  if (!h) return fail(TX_ERR_INVALID, "null Texelator handle");
  if (!embed || !token || !residual_out || !weight) return fail(TX_ERR_INVALID, "linear_split_embed_norm: null pointer");
  if (vocab <= 0) return fail(TX_ERR_INVALID, "linear_split_embed_norm: vocab must be positive");
  if (reinterpret_cast<uintptr_t>(embed) % 16 || reinterpret_cast<uintptr_t>(residual_out) % 16 ||
      reinterpret_cast<uintptr_t>(weight) % 16)
    return fail(TX_ERR_INVALID, "linear_split_embed_norm: table, residual and weight must be 16-byte aligned");
  if (h->bias && h->bias_dtype != TX_DTYPE_BF16) return fail(TX_ERR_INVALID, "linear_split_embed_norm: the bias must be BF16");
  const int64_t reads = (int64_t)h->RG * h->gemv_splits * h->K * 4;
  if (h->lut || h->K > tx::kNormMaxHidden || reads > kNormReadBudget)
    return fail(TX_ERR_UNSUPPORTED, "linear_split_embed_norm: the normalization does not fit the GEMV (LUT handle, "
                                    "K above 2048, or too many workgroups); gather, tx_add_rmsnorm and tx_linear_split");
  tx::GemvParams p{};
  p.tiles = h->tiles;
  p.scales = h->scales;
  p.M = h->M;
  p.K = h->K;
  p.Mp = h->Mp;
  p.RG = h->RG;
  p.CG = h->CG;
  p.tokens = 1;
  p.ks = h->gemv_splits;
  p.partials = h->partials;
  p.force_partials = 1;
  p.norm_embed = static_cast<const uint16_t *>(embed);
  p.norm_token = token;
  p.norm_vocab = vocab;
  p.norm_h_out = residual_out;
  p.norm_weight = static_cast<const uint16_t *>(weight);
  p.norm_eps = eps;
  DeviceGuard guard(h->device);
  TX_HIP(tx::launch_gemv(p, h->lookahead, true, reinterpret_cast<hipStream_t>(stream)));
  return TX_OK;
}

int tx_linear_swiglu_norm(uint64_t value, const float *residual_in, float *residual_out, uint64_t delta_handle,
                          const void *weight, float eps, void *out, void *stream) {
  g_last_error.clear();
  Handle *h = as_handle(value);
  if (!h) return fail(TX_ERR_INVALID, "null Texelator handle");
  if (!out) return fail(TX_ERR_INVALID, "linear_swiglu_norm: null output pointer");
  if (h->M % 32 != 0) return fail(TX_ERR_INVALID, "linear_swiglu_norm: the handle must hold [gate | up] with 16-row aligned halves");
  if (h->gemv_splits != 1 || h->CG > tx::kGemvMaxLdsColumns || h->lut)
    return fail(TX_ERR_UNSUPPORTED, "linear_swiglu_norm: needs a one-split, non-LUT handle with K <= 16384");
  if (h->bias && h->bias_dtype != TX_DTYPE_BF16) return fail(TX_ERR_INVALID, "linear_swiglu_norm: the bias must be BF16");
  tx::GemvParams p{};
  p.tiles = h->tiles;
  p.scales = h->scales;
  p.bias = h->bias;
  p.y = out;
  p.M = h->M;
  p.K = h->K;
  p.Mp = h->Mp;
  p.RG = h->RG;
  p.CG = h->CG;
  p.ks = 1;
  p.tokens = 1;
  const int status = set_norm_source(p, h, as_handle(delta_handle), residual_in, residual_out, weight, eps,
                                     (int64_t)h->RG / 2, "linear_swiglu_norm");
  if (status != TX_OK) return status;
  DeviceGuard guard(h->device);
  TX_HIP(tx::launch_gemv_swiglu(p, h->lookahead, reinterpret_cast<hipStream_t>(stream)));
  return TX_OK;
}

int tx_rope_kv_cache_split(uint64_t qkv_handle, const int64_t *positions, const float *cos_table, const float *sin_table,
                           int heads, int kv_heads, int head_dim, void *q_out, void *k_cache, void *v_cache,
                           int64_t max_context, void *stream) {
  g_last_error.clear();
  Handle *h = as_handle(qkv_handle);
  if (!h) return fail(TX_ERR_INVALID, "null Texelator handle");
  if (!positions || !cos_table || !sin_table || !q_out || !k_cache || !v_cache)
    return fail(TX_ERR_INVALID, "rope_kv_cache_split: null pointer");
  if (heads <= 0 || kv_heads <= 0 || head_dim <= 0 || head_dim % 2 || head_dim > 1024 || max_context <= 0 ||
      (int64_t)h->M < (int64_t)(heads + 2 * kv_heads) * head_dim)
    return fail(TX_ERR_INVALID, "rope_kv_cache_split: invalid shape");
  if (h->bias && h->bias_dtype != TX_DTYPE_BF16) return fail(TX_ERR_INVALID, "rope_kv_cache_split: the bias must be BF16");
  DeviceGuard guard(h->device);
  TX_HIP(tx::launch_rope_cache_split(split_source(h), 1, positions, cos_table, sin_table, heads, kv_heads, head_dim,
                                     static_cast<uint16_t *>(q_out), static_cast<uint16_t *>(k_cache),
                                     static_cast<uint16_t *>(v_cache), max_context, reinterpret_cast<hipStream_t>(stream)));
  return TX_OK;
}

int tx_rope_kv_cache(const void *qkv, int64_t row_stride, int64_t tokens, const int64_t *positions, const float *cos_table,
                     const float *sin_table, int heads, int kv_heads, int head_dim, void *q_out, void *k_cache,
                     void *v_cache, int64_t max_context, void *stream) {
  g_last_error.clear();
  if (!qkv || !positions || !cos_table || !sin_table || !q_out || !k_cache || !v_cache)
    return fail(TX_ERR_INVALID, "rope_kv_cache: null pointer");
  if (heads <= 0 || kv_heads <= 0 || head_dim <= 0 || head_dim % 2 || head_dim > 1024 || tokens < 0 ||
      row_stride < (int64_t)(heads + 2 * kv_heads) * head_dim || max_context <= 0)
    return fail(TX_ERR_INVALID, "rope_kv_cache: invalid shape");
  if (tokens == 0) return TX_OK;
  TX_HIP(tx::launch_rope_cache(static_cast<const uint16_t *>(qkv), row_stride, tokens, positions, cos_table, sin_table,
                               heads, kv_heads, head_dim, static_cast<uint16_t *>(q_out), static_cast<uint16_t *>(k_cache),
                               static_cast<uint16_t *>(v_cache), max_context, reinterpret_cast<hipStream_t>(stream)));
  return TX_OK;
}

int tx_decode_attention_workspace(int heads, int64_t length, int64_t *bytes) {
  g_last_error.clear();
  if (!bytes || heads <= 0 || length <= 0) return fail(TX_ERR_INVALID, "decode_attention_workspace: invalid arguments");
  *bytes = tx::decode_attention_workspace(heads, length);
  return TX_OK;
}

int tx_decode_attention(const void *q, const void *k_cache, const void *v_cache, const int64_t *position, int64_t length,
                        int heads, int kv_heads, int head_dim, int64_t max_context, float scale, void *workspace,
                        int64_t workspace_bytes, void *out, void *stream) {
  g_last_error.clear();
  if (!q || !k_cache || !v_cache || !position || !out || !workspace)
    return fail(TX_ERR_INVALID, "decode_attention: null pointer");
  if (!tx::decode_attention_supported(heads, kv_heads, head_dim))
    return fail(TX_ERR_UNSUPPORTED, "decode_attention: needs head_dim 128 and at most 8 query heads per KV head");
  if (length <= 0 || length > max_context || length > tx::decode_attention_max_length())
    return fail(TX_ERR_INVALID, "decode_attention: length outside the cache or above 65536");
  int64_t need = 0;
  tx_decode_attention_workspace(heads, length, &need);
  if (workspace_bytes < need) return fail(TX_ERR_INVALID, "decode_attention: workspace too small");
  TX_HIP(tx::launch_decode_attention(static_cast<const uint16_t *>(q), static_cast<const uint16_t *>(k_cache),
                                     static_cast<const uint16_t *>(v_cache), position, length, heads, kv_heads,
                                     max_context, scale, static_cast<float *>(workspace), static_cast<uint16_t *>(out),
                                     reinterpret_cast<hipStream_t>(stream)));
  return TX_OK;
}

int tx_prefill_attention(const void *q, int64_t q_stride, const void *k_cache, const void *v_cache, int64_t tokens,
                         int heads, int kv_heads, int head_dim, int64_t max_context, float scale, void *out,
                         int64_t out_stride, void *stream) {
  g_last_error.clear();
  if (!q || !k_cache || !v_cache || !out) return fail(TX_ERR_INVALID, "prefill_attention: null pointer");
  if (!tx::prefill_attention_supported(heads, kv_heads, head_dim))
    return fail(TX_ERR_UNSUPPORTED, "prefill_attention: needs head_dim 128 and heads a multiple of kv_heads");
  if (tokens <= 0) return TX_OK;
  if (tokens > max_context) return fail(TX_ERR_INVALID, "prefill_attention: more tokens than the cache holds");
  if (tokens > (int64_t)65535 * 64) return fail(TX_ERR_INVALID, "prefill_attention: token grid exceeds the launch limit");
  if (q_stride < (int64_t)heads * head_dim || out_stride < (int64_t)heads * head_dim || q_stride % 8 != 0 ||
      reinterpret_cast<uintptr_t>(q) % 16 != 0)
    return fail(TX_ERR_INVALID, "prefill_attention: q rows must be 16-byte aligned and hold heads * head_dim values");
  TX_HIP(tx::launch_prefill_attention(static_cast<const uint16_t *>(q), q_stride, static_cast<const uint16_t *>(k_cache),
                                      static_cast<const uint16_t *>(v_cache), tokens, heads, kv_heads, max_context, scale,
                                      static_cast<uint16_t *>(out), out_stride, reinterpret_cast<hipStream_t>(stream)));
  return TX_OK;
}

int tx_decode_attention_split(uint64_t qkv_handle, const int64_t *position, const float *rope_row, int64_t length,
                              int heads, int kv_heads, int head_dim, void *k_cache, void *v_cache,
                              int64_t max_context, float scale, void *workspace, int64_t workspace_bytes, void *out,
                              void *stream) {
  g_last_error.clear();
  Handle *h = as_handle(qkv_handle);
  if (!h) return fail(TX_ERR_INVALID, "null Texelator handle");
  if (!position || !rope_row || !k_cache || !v_cache || !out || !workspace)
    return fail(TX_ERR_INVALID, "decode_attention_split: null pointer");
  if (!tx::decode_attention_supported(heads, kv_heads, head_dim))
    return fail(TX_ERR_UNSUPPORTED, "decode_attention_split: needs head_dim 128 and at most 8 query heads per KV head");
  if ((int64_t)h->M < (int64_t)(heads + 2 * kv_heads) * head_dim)
    return fail(TX_ERR_INVALID, "decode_attention_split: qkv handle too narrow for the heads");
  if (h->bias && h->bias_dtype != TX_DTYPE_BF16) return fail(TX_ERR_INVALID, "decode_attention_split: the bias must be BF16");
  if (length <= 0 || length > max_context || length > tx::decode_attention_max_length())
    return fail(TX_ERR_INVALID, "decode_attention_split: length outside the cache or above 65536");
  int64_t need = 0;
  tx_decode_attention_workspace(heads, length, &need);
  if (workspace_bytes < need) return fail(TX_ERR_INVALID, "decode_attention_split: workspace too small");
  DeviceGuard guard(h->device);
  TX_HIP(tx::launch_decode_attention_split(split_source(h), position, rope_row, length, heads, kv_heads,
                                           static_cast<uint16_t *>(k_cache), static_cast<uint16_t *>(v_cache),
                                           max_context, scale, static_cast<float *>(workspace),
                                           static_cast<uint16_t *>(out), reinterpret_cast<hipStream_t>(stream)));
  return TX_OK;
}

int tx_decode_attention_o_split(uint64_t qkv_handle, uint64_t o_handle, const int64_t *position, const float *rope_row,
                                int64_t length, int heads, int kv_heads, int head_dim, void *k_cache, void *v_cache,
                                int64_t max_context, float scale, void *workspace, int64_t workspace_bytes,
                                void *stream) {
  g_last_error.clear();
  Handle *h = as_handle(qkv_handle);
  Handle *o = as_handle(o_handle);
  if (!h || !o) return fail(TX_ERR_INVALID, "null Texelator handle");
  if (!position || !rope_row || !k_cache || !v_cache || !workspace)
    return fail(TX_ERR_INVALID, "decode_attention_o_split: null pointer");
  if (!tx::decode_attention_supported(heads, kv_heads, head_dim))
    return fail(TX_ERR_UNSUPPORTED, "decode_attention_o_split: needs head_dim 128 and at most 8 query heads per KV head");
  if ((int64_t)h->M < (int64_t)(heads + 2 * kv_heads) * head_dim)
    return fail(TX_ERR_INVALID, "decode_attention_o_split: qkv handle too narrow for the heads");
  if (o->K != heads * head_dim) return fail(TX_ERR_INVALID, "decode_attention_o_split: o handle K must be heads * head_dim");
  if (o->device != h->device) return fail(TX_ERR_INVALID, "decode_attention_o_split: handles on different devices");
  if ((h->bias && h->bias_dtype != TX_DTYPE_BF16) || (o->bias && o->bias_dtype != TX_DTYPE_BF16))
    return fail(TX_ERR_INVALID, "decode_attention_o_split: biases must be BF16");
  if (length <= 0 || length > max_context || length > tx::decode_attention_max_length())
    return fail(TX_ERR_INVALID, "decode_attention_o_split: length outside the cache or above 65536");
  int64_t need = 0;
  tx_decode_attention_workspace(heads, length, &need);
  if (workspace_bytes < need) return fail(TX_ERR_INVALID, "decode_attention_o_split: workspace too small");
  // Each o workgroup merges the heads of its K split from every chunk: worth it while that is small.
  const int chunks = tx::decode_attention_chunks(length);
  const int heads_per_split = (o->CG + o->gemv_splits - 1) / o->gemv_splits;
  if (o->lut || chunks > tx::kMergeMaxChunks || heads_per_split * chunks > kMergeMaxChunkHeads)
    return fail(TX_ERR_UNSUPPORTED, "decode_attention_o_split: the merge does not fit the o GEMV (LUT handle, more "
                                    "than 16 chunks, or too many heads per split); use tx_decode_attention_split + "
                                    "tx_linear_split");
  DeviceGuard guard(h->device);
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  float *partials = static_cast<float *>(workspace);
  TX_HIP(tx::launch_decode_attention_split_partials(split_source(h), position, rope_row, length, heads, kv_heads,
                                                    static_cast<uint16_t *>(k_cache), static_cast<uint16_t *>(v_cache),
                                                    max_context, scale, partials, s));
  tx::GemvParams p{};
  p.tiles = o->tiles;
  p.scales = o->scales;
  p.M = o->M;
  p.K = o->K;
  p.Mp = o->Mp;
  p.RG = o->RG;
  p.CG = o->CG;
  p.tokens = 1;
  p.ks = o->gemv_splits;
  p.partials = o->partials;
  p.force_partials = 1;
  p.attn = partials;
  p.attn_chunks = chunks;
  p.attn_group = heads / kv_heads;
  TX_HIP(tx::launch_gemv(p, o->lookahead, true, s));
  return TX_OK;
}

int tx_lm_head_argmax_workspace(int64_t *bytes) {
  g_last_error.clear();
  if (!bytes) return fail(TX_ERR_INVALID, "lm_head_argmax_workspace: null output");
  *bytes = tx::lm_head_argmax_workspace();
  return TX_OK;
}

int tx_lm_head_argmax(const void *weight, int64_t vocab, int64_t hidden, const void *x, void *logits, void *workspace,
                      int64_t workspace_bytes, int64_t *token, void *stream) {
  g_last_error.clear();
  if (!weight || !x || !token || !workspace) return fail(TX_ERR_INVALID, "lm_head_argmax: null pointer");
  if (vocab <= 0 || vocab > 0x7FFFFFFF || hidden <= 0 || hidden > 16384 || hidden % 128)
    return fail(TX_ERR_INVALID, "lm_head_argmax: vocab must be 1..2^31-1 and hidden a multiple of 128 up to 16384");
  if (workspace_bytes < tx::lm_head_argmax_workspace() || reinterpret_cast<uintptr_t>(workspace) % 16 != 0)
    return fail(TX_ERR_INVALID, "lm_head_argmax: workspace missing or too small (see tx_lm_head_argmax_workspace)");
  if (reinterpret_cast<uintptr_t>(weight) % 16 != 0 || reinterpret_cast<uintptr_t>(x) % 16 != 0)
    return fail(TX_ERR_INVALID, "lm_head_argmax: weight and x must be 16-byte aligned");
  TX_HIP(tx::launch_lm_head_argmax(static_cast<const uint16_t *>(weight), vocab, (int)hidden, static_cast<const uint16_t *>(x),
                                   static_cast<uint16_t *>(logits), workspace, token, reinterpret_cast<hipStream_t>(stream)));
  return TX_OK;
}

int tx_swiglu(const void *gate_up, int64_t rows, int64_t intermediate, void *out, void *stream) {
  g_last_error.clear();
  if (!gate_up || !out || rows < 0 || intermediate <= 0 || intermediate % 8)
    return fail(TX_ERR_INVALID, "swiglu: intermediate size must be a positive multiple of 8");
  if (rows == 0) return TX_OK;
  TX_HIP(tx::launch_swiglu(static_cast<const uint16_t *>(gate_up), rows, intermediate, static_cast<uint16_t *>(out),
                           reinterpret_cast<hipStream_t>(stream)));
  return TX_OK;
}

int tx_kv_cache_append(const void *k, const void *v, int kv_heads, int head_dim, void *keys, void *values,
                       int64_t max_len, int64_t *length, void *stream) {
  g_last_error.clear();
  if (!k || !v || !keys || !values || !length) return fail(TX_ERR_INVALID, "kv_cache_append: null pointer");
  if (kv_heads <= 0 || head_dim <= 0 || max_len <= 0 || (int64_t)kv_heads * head_dim > (1 << 24) ||
      (int64_t)kv_heads * max_len * head_dim > (int64_t)1 << 40)
    return fail(TX_ERR_INVALID, "kv_cache_append: bad shape");
  if (reinterpret_cast<uintptr_t>(length) % 8) return fail(TX_ERR_INVALID, "kv_cache_append: length must be 8-byte aligned");
  TX_HIP(tx::launch_kv_append(static_cast<const uint16_t *>(k), static_cast<const uint16_t *>(v), kv_heads, head_dim,
                              static_cast<uint16_t *>(keys), static_cast<uint16_t *>(values), max_len, length,
                              reinterpret_cast<hipStream_t>(stream)));
  return TX_OK;
}

int tx_rope_rotate_half(const void *q, const void *k, int64_t tokens, int heads, int kv_heads, int head_dim,
                        const void *cos, const void *sin, void *q_out, void *k_out, void *stream) {
  g_last_error.clear();
  if (!q || !k || !cos || !sin || !q_out || !k_out) return fail(TX_ERR_INVALID, "rope_rotate_half: null pointer");
  if (tokens < 0 || heads <= 0 || kv_heads <= 0 || head_dim <= 0 || head_dim % 2 || head_dim > 512 ||
      tokens > 0x7FFFFFFF || heads + kv_heads > 65535)
    return fail(TX_ERR_INVALID, "rope_rotate_half: bad shape (head_dim even and at most 512)");
  if (tokens == 0) return TX_OK;
  TX_HIP(tx::launch_rope_rotate_half(static_cast<const uint16_t *>(q), static_cast<const uint16_t *>(k), tokens, heads,
                                     kv_heads, head_dim, static_cast<const uint16_t *>(cos),
                                     static_cast<const uint16_t *>(sin), static_cast<uint16_t *>(q_out),
                                     static_cast<uint16_t *>(k_out), reinterpret_cast<hipStream_t>(stream)));
  return TX_OK;
}

}  // extern "C"
