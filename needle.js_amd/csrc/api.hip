// C ABI of libneedle_hip.so: argument validation, HBM ownership, staging of
// host buffers, and dispatch to the kernels.  Validation mirrors the
// reference's invariants (backends/cq.ts:113-126, model/runtime.ts:150-160,
// 289-299, 885-891) so that the host binding can raise the same NeedleError
// codes.
#include <atomic>
#include <cmath>
#include <cstdarg>
#include <cstring>
#include <mutex>
#include <vector>

#include "nd_internal.hpp"

static thread_local std::string g_create_error;

nd_status nd_fail(nd_ctx* ctx, nd_status code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof buf, fmt, ap);
  va_end(ap);
  if (ctx) ctx->error = buf;
  else g_create_error = buf;
  return code;
}

nd_status nd_hip_fail(nd_ctx* ctx, hipError_t err, const char* what) {
  return nd_fail(ctx, err == hipErrorOutOfMemory ? ND_ERR_NOMEM : ND_ERR_BACKEND, "%s: %s (%d)",
                 what, hipGetErrorString(err), (int)err);
}

static nd_status ensure_stage(nd_ctx* ctx, size_t bytes) {
  if (ctx->stage_bytes >= bytes) return ND_OK;
  if (ctx->stage) {
    ND_HIP(ctx, hipStreamSynchronize(ctx->stream));
    ND_HIP(ctx, hipFree(ctx->stage));
    ctx->stage = nullptr;
    ctx->stage_bytes = 0;
  }
  size_t want = bytes < (1u << 20) ? (1u << 20) : bytes;
  ND_HIP(ctx, hipMalloc(&ctx->stage, want));
  ctx->stage_bytes = want;
  return ND_OK;
}

static nd_status ensure_host_stage(nd_ctx* ctx, size_t bytes) {
  if (ctx->host_stage_bytes >= bytes) return ND_OK;
  if (ctx->host_stage) {
    ND_HIP(ctx, hipStreamSynchronize(ctx->stream));
    ND_HIP(ctx, hipHostFree(ctx->host_stage));
    ctx->host_stage = nullptr;
    ctx->host_stage_bytes = 0;
  }
  size_t want = bytes < (64u << 10) ? (64u << 10) : bytes;
  ND_HIP(ctx, hipHostMalloc(&ctx->host_stage, want, hipHostMallocDefault));
  ctx->host_stage_bytes = want;
  return ND_OK;
}

static nd_status ensure_partials(nd_ctx* ctx, size_t floats) {
  if (ctx->attn_partial_floats >= floats) return ND_OK;
  if (ctx->attn_partials) {
    ND_HIP(ctx, hipStreamSynchronize(ctx->stream));
    ND_HIP(ctx, hipFree(ctx->attn_partials));
    ctx->attn_partials = nullptr;
    ctx->attn_partial_floats = 0;
  }
  ND_HIP(ctx, hipMalloc(&ctx->attn_partials, floats * sizeof(float)));
  ctx->attn_partial_floats = floats;
  if (!ctx->attn_counters) {
    const size_t cbytes = (size_t)kMaxAttentionKvHeads * kAttnCounterStride * sizeof(uint32_t);
    ND_HIP(ctx, hipMalloc(&ctx->attn_counters, cbytes));
    ND_HIP(ctx, hipMemsetAsync(ctx->attn_counters, 0, cbytes, ctx->stream));
    ND_HIP(ctx, hipStreamSynchronize(ctx->stream));
  }
  return ND_OK;
}

static inline size_t align256(size_t n) { return (n + 255) & ~size_t(255); }

// ------------------------------------------------------ workgroup placement

namespace {
// Thread 0 of workgroup L writes the id of the XCC (XCD) it runs on:
// HW_REG_XCC_ID (hardware register 20), bits [3:0].
__global__ void xcc_probe_kernel(uint32_t* out, uint32_t n) {
  if (threadIdx.x == 0 && blockIdx.x < n)
    out[blockIdx.x] = (uint32_t)__builtin_amdgcn_s_getreg((3 << 11) | (0 << 6) | 20) & 15u;
}

std::mutex g_xcd_mu;
int g_xcd_probed = -1;  // -1 no device probed yet, else 1 when every probed device passed
std::atomic<bool> g_xcd_local{false};
std::atomic<bool> g_xcd_off{false};
}  // namespace

hipError_t nd_probe_xcd_placement(hipStream_t s, bool* ok) {
  constexpr uint32_t kMax = 1024;
  uint32_t* d = nullptr;
  hipError_t e = hipMalloc(&d, kMax * sizeof(uint32_t));
  if (e != hipSuccess) return e;
  std::vector<uint32_t> h(kMax);
  bool pass = true;
  for (uint32_t n : {8u, 64u, kMax}) {
    hipLaunchKernelGGL(xcc_probe_kernel, dim3(n), dim3(64), 0, s, d, n);
    if ((e = hipGetLastError()) != hipSuccess) break;
    if ((e = hipMemcpyAsync(h.data(), d, n * sizeof(uint32_t), hipMemcpyDeviceToHost, s)) !=
        hipSuccess)
      break;
    if ((e = hipStreamSynchronize(s)) != hipSuccess) break;
    for (uint32_t L = 8; L < n; ++L) pass = pass && h[L] == h[L % 8];
  }
  hipFree(d);
  if (e != hipSuccess) return e;
  *ok = pass;
  std::lock_guard<std::mutex> lock(g_xcd_mu);
  g_xcd_probed = (g_xcd_probed != 0 && pass) ? 1 : 0;
  g_xcd_local = g_xcd_probed == 1 && !g_xcd_off;
  return hipSuccess;
}

bool nd_xcd_local() { return g_xcd_local.load(std::memory_order_relaxed); }

void nd_xcd_override(bool off) {
  std::lock_guard<std::mutex> lock(g_xcd_mu);
  g_xcd_off = off;
  g_xcd_local = g_xcd_probed == 1 && !off;
}

static void free_mat_buffers(nd_mat* m) {
  hipFree(m->w);
  hipFree(m->scales);
  hipFree(m->packed);
  hipFree(m->norms);
  delete m;
}

extern "C" {

nd_status nd_create(int32_t device, nd_ctx** out) {
  if (!out) return nd_fail(nullptr, ND_ERR_INVALID, "nd_create: out is NULL");
  *out = nullptr;
  int count = 0;
  hipError_t e = hipGetDeviceCount(&count);
  if (e != hipSuccess || count == 0)
    return nd_fail(nullptr, ND_ERR_BACKEND, "no HIP device is available (%s)",
                   hipGetErrorString(e));
  if (device < 0 || device >= count)
    return nd_fail(nullptr, ND_ERR_INVALID, "device %d is outside [0, %d)", device, count);
  e = hipSetDevice(device);
  if (e != hipSuccess)
    return nd_fail(nullptr, ND_ERR_BACKEND, "hipSetDevice(%d): %s", device, hipGetErrorString(e));
  hipDeviceProp_t prop;
  e = hipGetDeviceProperties(&prop, device);
  if (e != hipSuccess)
    return nd_fail(nullptr, ND_ERR_BACKEND, "hipGetDeviceProperties: %s", hipGetErrorString(e));
  if (std::strncmp(prop.gcnArchName, "gfx950", 6) != 0)
    return nd_fail(nullptr, ND_ERR_BACKEND, "device %d is %s; this library is built for gfx950",
                   device, prop.gcnArchName);
  nd_ctx* ctx = new nd_ctx();
  ctx->device = device;
  e = hipStreamCreateWithFlags(&ctx->stream, hipStreamNonBlocking);
  if (e != hipSuccess) {
    delete ctx;
    return nd_fail(nullptr, ND_ERR_BACKEND, "hipStreamCreate: %s", hipGetErrorString(e));
  }
  // The fixed attention scratch of nd_attention_static_d, once per device.
  e = nd_attention_scratch_setup(device);
  if (e != hipSuccess) {
    hipStreamDestroy(ctx->stream);
    delete ctx;
    return nd_fail(nullptr, ND_ERR_BACKEND, "attention scratch set-up on device %d: %s", device,
                   hipGetErrorString(e));
  }
  // Whether workgroups of one L % 8 share an XCD on this device (the
  // XCD-local hand-offs; otherwise their agent-scope forms run).
  bool placed = false;
  e = nd_probe_xcd_placement(ctx->stream, &placed);
  if (e != hipSuccess) {
    hipStreamDestroy(ctx->stream);
    delete ctx;
    return nd_fail(nullptr, ND_ERR_BACKEND, "workgroup placement probe on device %d: %s", device,
                   hipGetErrorString(e));
  }
  ctx->xcd_local = placed;
  e = hipMalloc(&ctx->mv_split, kMatvecSplitBytes);
  if (e == hipSuccess) e = hipMemsetAsync(ctx->mv_split, 0, kMatvecSplitBytes, ctx->stream);
  if (e == hipSuccess) e = hipStreamSynchronize(ctx->stream);
  if (e != hipSuccess) {
    if (ctx->mv_split) hipFree(ctx->mv_split);
    hipStreamDestroy(ctx->stream);
    delete ctx;
    return nd_fail(nullptr, ND_ERR_BACKEND, "hipMalloc(matvec split): %s", hipGetErrorString(e));
  }
  *out = ctx;
  return ND_OK;
}

nd_status nd_destroy(nd_ctx* ctx) {
  if (!ctx) return ND_OK;
  hipSetDevice(ctx->device);
  hipStreamSynchronize(ctx->stream);
  for (nd_mat* m : ctx->mats) free_mat_buffers(m);
  for (nd_kv* kv : ctx->kvs) {
    hipFree(kv->k);
    delete kv;
  }
  for (nd_pieces* pc : ctx->pieces) {
    hipFree(pc->offsets);
    delete pc;
  }
  for (nd_grammar* g : ctx->grammars) {
    hipFree(g->words);
    delete g;
  }
  if (ctx->stage) hipFree(ctx->stage);
  if (ctx->host_stage) hipHostFree(ctx->host_stage);
  if (ctx->attn_partials) hipFree(ctx->attn_partials);
  if (ctx->attn_counters) hipFree(ctx->attn_counters);
  if (ctx->mm_scratch) hipFree(ctx->mm_scratch);
  if (ctx->sel_split) hipFree(ctx->sel_split);
  if (ctx->mv_split) hipFree(ctx->mv_split);
  if (ctx->cq_prepared) hipFree(ctx->cq_prepared);
  hipStreamDestroy(ctx->stream);
  delete ctx;
  return ND_OK;
}

const char* nd_last_error(const nd_ctx* ctx) {
  return ctx ? ctx->error.c_str() : g_create_error.c_str();
}

nd_status nd_sync(nd_ctx* ctx) {
  if (!ctx) return nd_fail(nullptr, ND_ERR_BACKEND, "context is NULL");
  ND_HIP(ctx, hipStreamSynchronize(ctx->stream));
  return ND_OK;
}

void* nd_stream(nd_ctx* ctx) { return ctx ? (void*)ctx->stream : nullptr; }

nd_status nd_test_xcd_local(nd_ctx* ctx, int32_t enable, uint32_t* probed) {
  if (!ctx) return nd_fail(nullptr, ND_ERR_BACKEND, "context is NULL");
  ND_HIP(ctx, hipStreamSynchronize(ctx->stream));
  nd_xcd_override(enable == 0);
  if (probed) {
    std::lock_guard<std::mutex> lock(g_xcd_mu);
    *probed = g_xcd_probed == 1 ? 1u : 0u;
  }
  return ND_OK;
}

// ------------------------------------------------------------- matrices

static nd_status check_mat_shape(nd_ctx* ctx, uint32_t n, uint32_t k, uint32_t g) {
  if (n == 0 || k == 0 || g == 0)
    return nd_fail(ctx, ND_ERR_INVALID, "matrix shape %ux%u with group %u is empty", n, k, g);
  if (k % g != 0 || g % 16 != 0)
    return nd_fail(ctx, ND_ERR_INVALID, "group size %u must divide k=%u and be a multiple of 16",
                   g, k);
  // The matvec kernel maps k / 16 segments onto a power-of-two lane count.
  const uint32_t segs = k / 16;
  if (k % 16 != 0 || (segs & (segs - 1)) != 0 || segs < 8 || segs > 512)
    return nd_fail(ctx, ND_ERR_INVALID, "k=%u must be 16 * 2^j with 128 <= k <= 8192", k);
  return ND_OK;
}

static nd_status upload(nd_ctx* ctx, const void* w, const void* s, uint32_t n, uint32_t k,
                        uint32_t g, hipMemcpyKind kind, nd_mat** out) {
  if (!ctx || !out || !w || !s) return nd_fail(ctx, ND_ERR_INVALID, "nd_mat_upload: NULL argument");
  *out = nullptr;
  nd_status st = check_mat_shape(ctx, n, k, g);
  if (st != ND_OK) return st;
  ND_HIP(ctx, hipSetDevice(ctx->device));
  nd_mat* m = new nd_mat();
  m->n = n;
  m->k = k;
  m->g = g;
  const size_t wb = (size_t)n * k, sb = (size_t)n * (k / g) * sizeof(float);
  hipError_t e = hipMalloc(&m->w, wb);
  if (e == hipSuccess) e = hipMalloc(&m->scales, sb);
  if (e == hipSuccess) e = hipMemcpyAsync(m->w, w, wb, kind, ctx->stream);
  if (e == hipSuccess) e = hipMemcpyAsync(m->scales, s, sb, kind, ctx->stream);
  if (e == hipSuccess) e = hipStreamSynchronize(ctx->stream);
  if (e != hipSuccess) {
    hipFree(m->w);
    hipFree(m->scales);
    delete m;
    return nd_hip_fail(ctx, e, "matrix upload");
  }
  ctx->mats.insert(m);
  *out = m;
  return ND_OK;
}

nd_status nd_mat_upload_i8(nd_ctx* ctx, const int8_t* w, const float* scales, uint32_t n,
                           uint32_t k, uint32_t g, nd_mat** out) {
  return upload(ctx, w, scales, n, k, g, hipMemcpyHostToDevice, out);
}

nd_status nd_mat_upload_i8_d(nd_ctx* ctx, const int8_t* w_dev, const float* scales_dev,
                             uint32_t n, uint32_t k, uint32_t g, nd_mat** out) {
  return upload(ctx, w_dev, scales_dev, n, k, g, hipMemcpyDeviceToDevice, out);
}

nd_status nd_mat_free(nd_ctx* ctx, nd_mat* m) {
  if (!ctx) return nd_fail(nullptr, ND_ERR_BACKEND, "context is NULL");
  if (!m) return ND_OK;
  if (!ctx->mats.erase(m)) return nd_fail(ctx, ND_ERR_INVALID, "matrix does not belong to context");
  ND_HIP(ctx, hipStreamSynchronize(ctx->stream));
  free_mat_buffers(m);
  return ND_OK;
}

// A Cactus-Quant record (model/cact.ts:346-396): shape [n][k], group g (a
// power of two), bits 2, 3, 4 or 5 (ternary, packed as 2-bit crumbs), rows
// of kpad = ceil(k / g) * g codes.  The kernels work in units of 32 codes:
// rows are stored kstore = kpad rounded up to 32 codes wide, the extra
// codes zero and their groups' norms zero (the rotated input is zero there
// too, so they add nothing); they also need g >= 8 and kstore <= 8192.
nd_status nd_mat_upload_cq(nd_ctx* ctx, const uint8_t* packed, const uint16_t* norms,
                           const float* codebook, uint32_t n, uint32_t k, uint32_t g,
                           uint32_t bits, nd_mat** out) {
  if (!ctx) return nd_fail(nullptr, ND_ERR_BACKEND, "context is NULL");
  if (!out || !packed || !norms || (bits != 5 && !codebook))
    return nd_fail(ctx, ND_ERR_INVALID, "nd_mat_upload_cq: NULL argument");
  *out = nullptr;
  if (n == 0 || k == 0) return nd_fail(ctx, ND_ERR_INVALID, "CQ matrix %ux%u is empty", n, k);
  if (g == 0 || (g & (g - 1)) != 0)
    return nd_fail(ctx, ND_ERR_UNSUPPORTED, "CQ matrix has non-power-of-two group %u", g);
  if (bits < 2 || bits > 5)
    return nd_fail(ctx, ND_ERR_UNSUPPORTED, "CQ matrix uses unsupported record width %u", bits);
  const uint64_t kpad = ((uint64_t)k + g - 1) / g * g, kstore = (kpad + 31) / 32 * 32;
  const uint32_t pb = bits == 5 ? 2 : bits;
  if ((kpad * pb) % 8 != 0)
    return nd_fail(ctx, ND_ERR_INVALID, "CQ matrix has a fractional packed row size");
  if (g < 8 || kstore > kCqMaxKpad)
    return nd_fail(ctx, ND_ERR_UNSUPPORTED,
                   "CQ matrix k=%u with group %u: this backend needs group >= 8 and at most %u "
                   "padded columns", k, g, kCqMaxKpad);
  ND_HIP(ctx, hipSetDevice(ctx->device));
  if (!ctx->cq_prepared)
    ND_HIP(ctx, hipMalloc(&ctx->cq_prepared, (size_t)kCqPreparedRows * kCqMaxKpad * sizeof(float)));
  nd_mat* m = new nd_mat();
  m->n = n;
  m->k = k;
  m->g = g;
  m->bits = bits;
  m->kpad = (uint32_t)kstore;
  m->row_bytes = (uint32_t)(kstore * pb / 8);
  if (bits == 5) {
    // cqMatvecPrepared's crumb table [0, c, 0, -c], c = 1.2240064 / sqrt(g)
    // (backends/cq.ts:182-184), rounded to fp32 once.
    const float c = (float)(1.2240064 / std::sqrt((double)g));
    m->cb[1] = c;
    m->cb[3] = -c;
  } else {
    for (uint32_t i = 0; i < (1u << bits); ++i) m->cb[i] = codebook[i];
  }
  const size_t pbytes = (size_t)n * m->row_bytes, nbytes = (size_t)n * (kstore / g) * 2;
  const void* psrc = packed;
  const void* nsrc = norms;
  std::vector<uint8_t> ppad;
  std::vector<uint16_t> npad;
  if (kstore != kpad) {  // widen each row to kstore codes: zero codes, zero norms
    const size_t src_row = kpad * pb / 8, src_groups = kpad / g, groups = kstore / g;
    ppad.assign(pbytes, 0);
    npad.assign((size_t)n * groups, 0);
    for (size_t r = 0; r < n; ++r) {
      std::memcpy(&ppad[r * m->row_bytes], packed + r * src_row, src_row);
      std::memcpy(&npad[r * groups], norms + r * src_groups, src_groups * 2);
    }
    psrc = ppad.data();
    nsrc = npad.data();
  }
  hipError_t e = hipMalloc(&m->packed, pbytes);
  if (e == hipSuccess) e = hipMalloc(&m->norms, nbytes);
  if (e == hipSuccess) e = hipMemcpyAsync(m->packed, psrc, pbytes, hipMemcpyHostToDevice, ctx->stream);
  if (e == hipSuccess) e = hipMemcpyAsync(m->norms, nsrc, nbytes, hipMemcpyHostToDevice, ctx->stream);
  if (e == hipSuccess) e = hipStreamSynchronize(ctx->stream);
  if (e != hipSuccess) {
    free_mat_buffers(m);
    return nd_hip_fail(ctx, e, "CQ matrix upload");
  }
  ctx->mats.insert(m);
  *out = m;
  return ND_OK;
}

nd_status nd_mat_cq_info(const nd_mat* m, uint32_t* bits, uint32_t* kpad, uint32_t* row_bytes) {
  if (!m) return ND_ERR_INVALID;
  if (bits) *bits = m->bits;
  if (kpad) *kpad = m->kpad;
  if (row_bytes) *row_bytes = m->row_bytes;
  return ND_OK;
}

nd_status nd_mat_info(const nd_mat* m, const int8_t** w_dev, const float** scales_dev, uint32_t* n,
                      uint32_t* k, uint32_t* g) {
  if (!m) return ND_ERR_INVALID;
  if (w_dev) *w_dev = m->w;
  if (scales_dev) *scales_dev = m->scales;
  if (n) *n = m->n;
  if (k) *k = m->k;
  if (g) *g = m->g;
  return ND_OK;
}

// --------------------------------------------------------------- matvec

// Either matrix form: int8 codes with scales, or Cactus-Quant.  y rows are
// y_stride floats apart.
static hipError_t launch_matvec_any(nd_ctx* ctx, const nd_mat* m, const float* x, uint32_t batch,
                                    uint32_t row_start, uint32_t row_count, float* y,
                                    uint32_t y_stride, hipStream_t s, void* split) {
  if (!m->bits) return nd_launch_matvec(m, x, batch, m->k, row_start, row_count, y, y_stride, s, split);
  return nd_launch_cq_matvec(m, x, batch, m->k, ctx->cq_prepared, row_start, row_count, y,
                             y_stride, s);
}

static nd_status check_range(nd_ctx* ctx, const nd_mat* m, uint32_t row_start, uint32_t row_count) {
  if (!m) return nd_fail(ctx, ND_ERR_INVALID, "matrix is NULL");
  if ((uint64_t)row_start + row_count > m->n)
    return nd_fail(ctx, ND_ERR_INVALID, "Invalid matrix row range %u:%llu", row_start,
                   (unsigned long long)row_start + row_count);
  return ND_OK;
}

nd_status nd_matvec_d(nd_ctx* ctx, const nd_mat* m, const float* x, uint32_t batch,
                      uint32_t row_start, uint32_t row_count, float* y, void* stream) {
  if (!ctx) return nd_fail(nullptr, ND_ERR_BACKEND, "context is NULL");
  nd_status st = check_range(ctx, m, row_start, row_count);
  if (st != ND_OK) return st;
  if ((batch && (!x || !y)) || (reinterpret_cast<uintptr_t>(x) & 15))
    return nd_fail(ctx, ND_ERR_INVALID, "x must be a 16-byte aligned device pointer");
  ND_HIP(ctx, launch_matvec_any(ctx, m, x, batch, row_start, row_count, y, row_count,
                                nd_pick_stream(ctx, stream), ctx->mv_split));
  return ND_OK;
}

nd_status nd_matvec_stamped_d(nd_ctx* ctx, const nd_mat* m, const float* x, uint32_t row_start,
                              uint32_t row_count, float* y, uint64_t* stamps, uint32_t capacity,
                              uint32_t* workgroups, void* stream) {
  if (!ctx) return nd_fail(nullptr, ND_ERR_BACKEND, "context is NULL");
  nd_status st = check_range(ctx, m, row_start, row_count);
  if (st != ND_OK) return st;
  if (m->bits || row_count == 0 || !x || !y || !stamps || !workgroups ||
      (reinterpret_cast<uintptr_t>(x) & 15))
    return nd_fail(ctx, ND_ERR_INVALID,
                   "nd_matvec_stamped_d: an int8 matrix, rows, a 16-byte aligned x, y, stamps "
                   "and workgroups");
  const hipError_t e = nd_launch_matvec_stamped(m, x, row_start, row_count, y, stamps, capacity,
                                                workgroups, nd_pick_stream(ctx, stream));
  if (e == hipErrorInvalidValue)
    return nd_fail(ctx, ND_ERR_INVALID, "nd_matvec_stamped_d: %u workgroups, room for %u stamps",
                   *workgroups, capacity);
  ND_HIP(ctx, e);
  return ND_OK;
}

nd_status nd_stream_read_d(nd_ctx* ctx, const void* src, uint64_t bytes, uint32_t blocks,
                           uint32_t* out, void* stream) {
  if (!ctx) return nd_fail(nullptr, ND_ERR_BACKEND, "context is NULL");
  if (!src || !out || bytes == 0 || (bytes & 15) || (reinterpret_cast<uintptr_t>(src) & 15) ||
      blocks == 0 || blocks > 65535)
    return nd_fail(ctx, ND_ERR_INVALID,
                   "nd_stream_read_d: 16-byte aligned source, bytes a nonzero multiple of 16, "
                   "1..65535 blocks");
  ND_HIP(ctx, nd_launch_stream_read(src, bytes, blocks, out, nd_pick_stream(ctx, stream)));
  return ND_OK;
}

nd_status nd_matvec(nd_ctx* ctx, const nd_mat* m, const float* x, uint32_t batch,
                    uint32_t row_start, uint32_t row_count, float* y) {
  if (!ctx) return nd_fail(nullptr, ND_ERR_BACKEND, "context is NULL");
  nd_status st = check_range(ctx, m, row_start, row_count);
  if (st != ND_OK) return st;
  if (batch == 0 || row_count == 0) return ND_OK;
  if (!x || !y) return nd_fail(ctx, ND_ERR_INVALID, "x or y is NULL");
  const size_t xb = (size_t)batch * m->k * sizeof(float);
  const size_t yb = (size_t)batch * row_count * sizeof(float);
  st = ensure_stage(ctx, align256(xb) + yb);
  if (st != ND_OK) return st;
  float* dx = reinterpret_cast<float*>(ctx->stage);
  float* dy = reinterpret_cast<float*>(reinterpret_cast<char*>(ctx->stage) + align256(xb));
  ND_HIP(ctx, hipMemcpyAsync(dx, x, xb, hipMemcpyHostToDevice, ctx->stream));
  ND_HIP(ctx, launch_matvec_any(ctx, m, dx, batch, row_start, row_count, dy, row_count,
                                ctx->stream, ctx->mv_split));
  ND_HIP(ctx, hipMemcpyAsync(y, dy, yb, hipMemcpyDeviceToHost, ctx->stream));
  ND_HIP(ctx, hipStreamSynchronize(ctx->stream));
  return ND_OK;
}

nd_status nd_matvec_batch(nd_ctx* ctx, const nd_matvec_job* jobs, uint32_t count) {
  if (!ctx) return nd_fail(nullptr, ND_ERR_BACKEND, "context is NULL");
  if (count == 0) return ND_OK;
  if (!jobs) return nd_fail(ctx, ND_ERR_INVALID, "jobs is NULL");
  size_t total = 0;
  for (uint32_t i = 0; i < count; ++i) {
    nd_status st = check_range(ctx, jobs[i].mat, jobs[i].row_start, jobs[i].row_count);
    if (st != ND_OK) return st;
    if (!jobs[i].x || (jobs[i].row_count && !jobs[i].y))
      return nd_fail(ctx, ND_ERR_INVALID, "job %u has a NULL buffer", i);
    total += align256((size_t)jobs[i].mat->k * 4) + align256((size_t)jobs[i].row_count * 4);
  }
  nd_status st = ensure_stage(ctx, total);
  if (st != ND_OK) return st;
  char* base = reinterpret_cast<char*>(ctx->stage);
  std::vector<float*> dys(count);
  size_t off = 0;
  // Identical host inputs are uploaded once (the reference prepares each
  // input once per geometry, backends/cpu.ts:18-26).
  std::vector<std::pair<const float*, float*>> seen;
  for (uint32_t i = 0; i < count; ++i) {
    const nd_mat* m = jobs[i].mat;
    float* dx = nullptr;
    for (auto& pr : seen)
      if (pr.first == jobs[i].x) dx = pr.second;
    if (!dx) {
      dx = reinterpret_cast<float*>(base + off);
      off += align256((size_t)m->k * 4);
      ND_HIP(ctx, hipMemcpyAsync(dx, jobs[i].x, (size_t)m->k * 4, hipMemcpyHostToDevice, ctx->stream));
      seen.emplace_back(jobs[i].x, dx);
    }
    dys[i] = reinterpret_cast<float*>(base + off);
    off += align256((size_t)jobs[i].row_count * 4);
    ND_HIP(ctx, launch_matvec_any(ctx, m, dx, 1, jobs[i].row_start, jobs[i].row_count, dys[i],
                                  jobs[i].row_count, ctx->stream, nullptr));
  }
  for (uint32_t i = 0; i < count; ++i)
    if (jobs[i].row_count)
      ND_HIP(ctx, hipMemcpyAsync(jobs[i].y, dys[i], (size_t)jobs[i].row_count * 4,
                                 hipMemcpyDeviceToHost, ctx->stream));
  ND_HIP(ctx, hipStreamSynchronize(ctx->stream));
  return ND_OK;
}

nd_status nd_row_d(nd_ctx* ctx, const nd_mat* m, uint32_t row, float* out, void* stream) {
  if (!ctx) return nd_fail(nullptr, ND_ERR_BACKEND, "context is NULL");
  if (!m || row >= m->n) return nd_fail(ctx, ND_ERR_INVALID, "Matrix row %u is out of range", row);
  if (!out) return nd_fail(ctx, ND_ERR_INVALID, "output is NULL");
  hipStream_t s = nd_pick_stream(ctx, stream);
  ND_HIP(ctx, m->bits ? nd_launch_cq_row(m, row, out, s) : nd_launch_row(m, row, out, s));
  return ND_OK;
}

nd_status nd_row(nd_ctx* ctx, const nd_mat* m, uint32_t row, float* out) {
  if (!ctx) return nd_fail(nullptr, ND_ERR_BACKEND, "context is NULL");
  if (!m || row >= m->n) return nd_fail(ctx, ND_ERR_INVALID, "Matrix row %u is out of range", row);
  if (!out) return nd_fail(ctx, ND_ERR_INVALID, "output is NULL");
  nd_status st = ensure_stage(ctx, (size_t)m->k * 4);
  if (st == ND_OK) st = ensure_host_stage(ctx, (size_t)m->k * 4);
  if (st != ND_OK) return st;
  float* d = reinterpret_cast<float*>(ctx->stage);
  ND_HIP(ctx, m->bits ? nd_launch_cq_row(m, row, d, ctx->stream) : nd_launch_row(m, row, d, ctx->stream));
  // Through pinned memory: a pageable destination costs a staged copy.
  ND_HIP(ctx, hipMemcpyAsync(ctx->host_stage, d, (size_t)m->k * 4, hipMemcpyDeviceToHost,
                             ctx->stream));
  ND_HIP(ctx, hipStreamSynchronize(ctx->stream));
  std::memcpy(out, ctx->host_stage, (size_t)m->k * 4);
  return ND_OK;
}

// ------------------------------------------------ batched matvec (MFMA)

static nd_status check_matmul(nd_ctx* ctx, const nd_mat* m) {
  if (!m) return nd_fail(ctx, ND_ERR_INVALID, "matrix is NULL");
  if (m->bits) return nd_fail(ctx, ND_ERR_INVALID, "nd_matmul needs an int8 matrix");
  if (m->g != m->k || m->k % 64 != 0 || m->k > 2048)
    return nd_fail(ctx, ND_ERR_INVALID,
                   "nd_matmul needs per-row scales (g == k), k %% 64 == 0 and k <= 2048 "
                   "(got k=%u g=%u)", m->k, m->g);
  return ND_OK;
}

static nd_status ensure_mm_scratch(nd_ctx* ctx, size_t bytes) {
  if (ctx->mm_scratch_bytes >= bytes) return ND_OK;
  if (ctx->mm_scratch) {
    ND_HIP(ctx, hipStreamSynchronize(ctx->stream));
    ND_HIP(ctx, hipFree(ctx->mm_scratch));
    ctx->mm_scratch = nullptr;
    ctx->mm_scratch_bytes = 0;
  }
  ND_HIP(ctx, hipMalloc(&ctx->mm_scratch, bytes));
  ctx->mm_scratch_bytes = bytes;
  return ND_OK;
}

nd_status nd_matmul_d(nd_ctx* ctx, const nd_mat* m, const float* x, uint32_t rows, float* y,
                      uint32_t accumulate, void* stream) {
  if (!ctx) return nd_fail(nullptr, ND_ERR_BACKEND, "context is NULL");
  nd_status st = check_matmul(ctx, m);
  if (st != ND_OK) return st;
  if (rows == 0) return ND_OK;
  if (!x || !y) return nd_fail(ctx, ND_ERR_INVALID, "x or y is NULL");
  const size_t dbytes = align256((size_t)3 * rows * m->k);
  st = ensure_mm_scratch(ctx, dbytes + align256((size_t)rows * 4));
  if (st != ND_OK) return st;
  int8_t* digits = reinterpret_cast<int8_t*>(ctx->mm_scratch);
  float* fm = reinterpret_cast<float*>(reinterpret_cast<char*>(ctx->mm_scratch) + dbytes);
  hipStream_t s = nd_pick_stream(ctx, stream);
  ND_HIP(ctx, nd_launch_digitize(x, m->k, nullptr, nullptr, digits, fm, rows, m->k, s));
  ND_HIP(ctx, nd_launch_gemm(m, digits, fm, y, m->n, rows, accumulate ? 1 : 0, s));
  return ND_OK;
}

nd_status nd_matmul(nd_ctx* ctx, const nd_mat* m, const float* x, uint32_t rows, float* y) {
  if (!ctx) return nd_fail(nullptr, ND_ERR_BACKEND, "context is NULL");
  nd_status st = check_matmul(ctx, m);
  if (st != ND_OK) return st;
  if (rows == 0) return ND_OK;
  if (!x || !y) return nd_fail(ctx, ND_ERR_INVALID, "x or y is NULL");
  const size_t xb = (size_t)rows * m->k * 4, yb = (size_t)rows * m->n * 4;
  st = ensure_stage(ctx, align256(xb) + yb);
  if (st != ND_OK) return st;
  float* dx = reinterpret_cast<float*>(ctx->stage);
  float* dy = reinterpret_cast<float*>(reinterpret_cast<char*>(ctx->stage) + align256(xb));
  ND_HIP(ctx, hipMemcpyAsync(dx, x, xb, hipMemcpyHostToDevice, ctx->stream));
  st = nd_matmul_d(ctx, m, dx, rows, dy, 0, ctx->stream);
  if (st != ND_OK) return st;
  ND_HIP(ctx, hipMemcpyAsync(y, dy, yb, hipMemcpyDeviceToHost, ctx->stream));
  ND_HIP(ctx, hipStreamSynchronize(ctx->stream));
  return ND_OK;
}

// -------------------------------------------------------------- KV cache

nd_status nd_kv_create(nd_ctx* ctx, uint32_t layers, uint32_t kv_heads, uint32_t head_dim,
                       uint32_t max_length, uint32_t sink, uint32_t window, uint32_t mode,
                       nd_kv** out) {
  if (!ctx) return nd_fail(nullptr, ND_ERR_BACKEND, "context is NULL");
  if (!out) return nd_fail(ctx, ND_ERR_INVALID, "out is NULL");
  *out = nullptr;
  if (head_dim != 64) return nd_fail(ctx, ND_ERR_INVALID, "head_dim %u is not 64", head_dim);
  if (layers == 0 || kv_heads == 0 || max_length == 0)
    return nd_fail(ctx, ND_ERR_INVALID, "empty KV cache geometry");
  if (kv_heads > kMaxAttentionKvHeads || max_length > kMaxAttentionPositions)
    return nd_fail(ctx, ND_ERR_INVALID, "KV cache limits: at most %u heads and %u positions",
                   kMaxAttentionKvHeads, kMaxAttentionPositions);
  if (mode != ND_KV_INT8 && mode != ND_KV_FLOAT32)
    return nd_fail(ctx, ND_ERR_INVALID, "unknown KV mode %u", mode);
  nd_kv* kv = new nd_kv();
  kv->layers = layers;
  kv->kv_heads = kv_heads;
  kv->head_dim = head_dim;
  kv->max_length = max_length;
  kv->sink = sink < max_length ? sink : max_length;
  kv->window = window;
  kv->alloc = window > 0 ? (max_length < kv->sink + window ? max_length : kv->sink + window)
                         : max_length;
  kv->mode = mode;
  const size_t rows = (size_t)layers * kv_heads * kv->alloc;
  const size_t code_bytes = rows * head_dim * (mode == ND_KV_FLOAT32 ? 4 : 1);
  const size_t scale_bytes = rows * sizeof(float);
  const size_t total = 2 * align256(code_bytes) + 2 * align256(scale_bytes);
  char* base = nullptr;
  hipError_t e = hipSetDevice(ctx->device);
  if (e == hipSuccess) e = hipMalloc(&base, total);
  if (e == hipSuccess) e = hipMemsetAsync(base, 0, total, ctx->stream);
  if (e == hipSuccess) e = hipStreamSynchronize(ctx->stream);
  if (e != hipSuccess) {
    if (base) hipFree(base);
    delete kv;
    return nd_hip_fail(ctx, e, "KV cache allocation");
  }
  kv->k = base;
  kv->v = base + align256(code_bytes);
  kv->ks = reinterpret_cast<float*>(base + 2 * align256(code_bytes));
  kv->vs = reinterpret_cast<float*>(base + 2 * align256(code_bytes) + align256(scale_bytes));
  // Attention partials for the largest visible set of this cache, with up to
  // 8 query heads per KV head.
  const uint32_t max_visible = kv->alloc;
  nd_status st = ensure_partials(ctx, nd_attention_partial_floats(kv_heads * 8, kv_heads, max_visible));
  if (st != ND_OK) {
    hipFree(base);
    delete kv;
    return st;
  }
  ctx->kvs.insert(kv);
  *out = kv;
  return ND_OK;
}

nd_status nd_kv_free(nd_ctx* ctx, nd_kv* kv) {
  if (!ctx) return nd_fail(nullptr, ND_ERR_BACKEND, "context is NULL");
  if (!kv) return ND_OK;
  if (!ctx->kvs.erase(kv)) return nd_fail(ctx, ND_ERR_INVALID, "cache does not belong to context");
  ND_HIP(ctx, hipStreamSynchronize(ctx->stream));
  hipFree(kv->k);
  delete kv;
  return ND_OK;
}

static size_t kv_total_bytes(const nd_kv* kv) {
  const size_t rows = (size_t)kv->layers * kv->kv_heads * kv->alloc;
  const size_t code_bytes = rows * kv->head_dim * (kv->mode == ND_KV_FLOAT32 ? 4 : 1);
  return 2 * align256(code_bytes) + 2 * align256(rows * sizeof(float));
}

nd_status nd_kv_clear(nd_ctx* ctx, nd_kv* kv) {
  if (!ctx) return nd_fail(nullptr, ND_ERR_BACKEND, "context is NULL");
  if (!kv) return nd_fail(ctx, ND_ERR_INVALID, "cache is NULL");
  ND_HIP(ctx, hipMemsetAsync(kv->k, 0, kv_total_bytes(kv), ctx->stream));
  return ND_OK;
}

nd_status nd_kv_info(const nd_kv* kv, uint32_t* alloc, void** k_codes, void** v_codes,
                     float** k_scales, float** v_scales) {
  if (!kv) return ND_ERR_INVALID;
  if (alloc) *alloc = kv->alloc;
  if (k_codes) *k_codes = kv->k;
  if (v_codes) *v_codes = kv->v;
  if (k_scales) *k_scales = kv->ks;
  if (v_scales) *v_scales = kv->vs;
  return ND_OK;
}

static nd_status check_store(nd_ctx* ctx, const nd_kv* kv, uint32_t layer, uint32_t position,
                             uint32_t count) {
  if (!kv) return nd_fail(ctx, ND_ERR_INVALID, "cache is NULL");
  if (layer >= kv->layers)
    return nd_fail(ctx, ND_ERR_INVALID, "layer %u is outside [0, %u)", layer, kv->layers);
  if ((uint64_t)position + count > kv->max_length)
    return nd_fail(ctx, ND_ERR_OVERFLOW, "Position %llu reached runtime limit %u",
                   (unsigned long long)position + count - 1, kv->max_length);
  return ND_OK;
}

nd_status nd_kv_store_d(nd_ctx* ctx, nd_kv* kv, uint32_t layer, uint32_t position, uint32_t count,
                        const float* k, const float* v, void* stream) {
  if (!ctx) return nd_fail(nullptr, ND_ERR_BACKEND, "context is NULL");
  nd_status st = check_store(ctx, kv, layer, position, count);
  if (st != ND_OK) return st;
  if (count && (!k || !v)) return nd_fail(ctx, ND_ERR_INVALID, "k or v is NULL");
  ND_HIP(ctx, nd_launch_kv_store(kv, layer, position, 0, count, k, v, nd_pick_stream(ctx, stream)));
  return ND_OK;
}

nd_status nd_kv_store(nd_ctx* ctx, nd_kv* kv, uint32_t layer, uint32_t position, uint32_t count,
                      const float* k, const float* v) {
  if (!ctx) return nd_fail(nullptr, ND_ERR_BACKEND, "context is NULL");
  nd_status st = check_store(ctx, kv, layer, position, count);
  if (st != ND_OK) return st;
  if (count == 0) return ND_OK;
  if (!k || !v) return nd_fail(ctx, ND_ERR_INVALID, "k or v is NULL");
  const size_t bytes = (size_t)count * kv->kv_heads * kv->head_dim * sizeof(float);
  st = ensure_stage(ctx, 2 * align256(bytes));
  if (st != ND_OK) return st;
  float* dk = reinterpret_cast<float*>(ctx->stage);
  float* dv = reinterpret_cast<float*>(reinterpret_cast<char*>(ctx->stage) + align256(bytes));
  ND_HIP(ctx, hipMemcpyAsync(dk, k, bytes, hipMemcpyHostToDevice, ctx->stream));
  ND_HIP(ctx, hipMemcpyAsync(dv, v, bytes, hipMemcpyHostToDevice, ctx->stream));
  ND_HIP(ctx, nd_launch_kv_store(kv, layer, position, 0, count, dk, dv, ctx->stream));
  ND_HIP(ctx, hipStreamSynchronize(ctx->stream));
  return ND_OK;
}

nd_status nd_kv_read(nd_ctx* ctx, const nd_kv* kv, uint32_t layer, uint32_t head, void* k_codes,
                     void* v_codes, float* k_scales, float* v_scales) {
  if (!ctx) return nd_fail(nullptr, ND_ERR_BACKEND, "context is NULL");
  if (!kv || layer >= kv->layers || head >= kv->kv_heads)
    return nd_fail(ctx, ND_ERR_INVALID, "layer/head outside the cache");
  const size_t row0 = ((size_t)layer * kv->kv_heads + head) * kv->alloc;
  const size_t esz = kv->mode == ND_KV_FLOAT32 ? 4 : 1;
  const size_t cb = (size_t)kv->alloc * kv->head_dim * esz;
  const char* kc = reinterpret_cast<const char*>(kv->k) + row0 * kv->head_dim * esz;
  const char* vc = reinterpret_cast<const char*>(kv->v) + row0 * kv->head_dim * esz;
  if (k_codes) ND_HIP(ctx, hipMemcpyAsync(k_codes, kc, cb, hipMemcpyDeviceToHost, ctx->stream));
  if (v_codes) ND_HIP(ctx, hipMemcpyAsync(v_codes, vc, cb, hipMemcpyDeviceToHost, ctx->stream));
  if (k_scales)
    ND_HIP(ctx, hipMemcpyAsync(k_scales, kv->ks + row0, kv->alloc * 4, hipMemcpyDeviceToHost, ctx->stream));
  if (v_scales)
    ND_HIP(ctx, hipMemcpyAsync(v_scales, kv->vs + row0, kv->alloc * 4, hipMemcpyDeviceToHost, ctx->stream));
  ND_HIP(ctx, hipStreamSynchronize(ctx->stream));
  return ND_OK;
}

static nd_status check_attention(nd_ctx* ctx, const nd_kv* kv, uint32_t layer, uint32_t position,
                                 uint32_t q_heads) {
  if (!kv) return nd_fail(ctx, ND_ERR_INVALID, "cache is NULL");
  if (layer >= kv->layers)
    return nd_fail(ctx, ND_ERR_INVALID, "layer %u is outside [0, %u)", layer, kv->layers);
  if (position >= kv->max_length)
    return nd_fail(ctx, ND_ERR_OVERFLOW, "Position %u reached runtime limit %u", position,
                   kv->max_length);
  const uint32_t rep = q_heads / kv->kv_heads;
  if (q_heads == 0 || q_heads % kv->kv_heads != 0 || (rep != 1 && rep != 2 && rep != 4 && rep != 8))
    return nd_fail(ctx, ND_ERR_INVALID,
                   "q_heads %u must be 1, 2, 4 or 8 times the %u KV heads", q_heads, kv->kv_heads);
  return ND_OK;
}

nd_status nd_attention_d(nd_ctx* ctx, const nd_kv* kv, uint32_t layer, uint32_t position,
                         const float* q, uint32_t q_heads, float* out, void* stream) {
  if (!ctx) return nd_fail(nullptr, ND_ERR_BACKEND, "context is NULL");
  nd_status st = check_attention(ctx, kv, layer, position, q_heads);
  if (st != ND_OK) return st;
  if (!q || !out || (reinterpret_cast<uintptr_t>(q) & 15))
    return nd_fail(ctx, ND_ERR_INVALID, "q must be a 16-byte aligned device pointer");
  const nd_visible vis = nd_kv_visible(kv, position);
  const size_t need = nd_attention_partial_floats(q_heads, kv->kv_heads, vis.count);
  if (need > ctx->attn_partial_floats && nd_attention_chunks(vis.count, kv->kv_heads) > 1)
    return nd_fail(ctx, ND_ERR_INVALID, "attention partials too small (%zu > %zu floats)", need,
                   ctx->attn_partial_floats);
  ND_HIP(ctx, nd_launch_attention(kv, layer, position, q, q_heads, out, ctx->attn_partials,
                                  ctx->attn_counters, nd_pick_stream(ctx, stream)));
  return ND_OK;
}

nd_status nd_attention_stamped_d(nd_ctx* ctx, const nd_kv* kv, uint32_t layer, uint32_t position,
                                 const float* q, uint32_t q_heads, float* out, uint64_t* stamps,
                                 uint32_t capacity, uint32_t* workgroups, void* stream) {
  if (!ctx) return nd_fail(nullptr, ND_ERR_BACKEND, "context is NULL");
  nd_status st = check_attention(ctx, kv, layer, position, q_heads);
  if (st != ND_OK) return st;
  if (!q || !out || !stamps || !workgroups || (reinterpret_cast<uintptr_t>(q) & 15))
    return nd_fail(ctx, ND_ERR_INVALID,
                   "nd_attention_stamped_d: a 16-byte aligned q, out, stamps and workgroups");
  const nd_visible vis = nd_kv_visible(kv, position);
  const size_t need = nd_attention_partial_floats(q_heads, kv->kv_heads, vis.count);
  if (need > ctx->attn_partial_floats)
    return nd_fail(ctx, ND_ERR_INVALID, "attention partials too small (%zu > %zu floats)", need,
                   ctx->attn_partial_floats);
  *workgroups = 0;
  const hipError_t e =
      nd_launch_attention(kv, layer, position, q, q_heads, out, ctx->attn_partials,
                          ctx->attn_counters, nd_pick_stream(ctx, stream), stamps, capacity,
                          workgroups);
  if (e == hipErrorInvalidValue)
    return nd_fail(ctx, ND_ERR_UNSUPPORTED,
                   "nd_attention_stamped_d: only the XCD-local one-tile form is stamped, and "
                   "%u workgroups need room for as many stamps (%u)", *workgroups, capacity);
  ND_HIP(ctx, e);
  return ND_OK;
}

nd_status nd_attention_static_d(nd_ctx* ctx, const nd_kv* kv, uint32_t layer, uint32_t position,
                                const float* q, uint32_t q_heads, float* out, void* stream) {
  if (!ctx) return nd_fail(nullptr, ND_ERR_BACKEND, "context is NULL");
  nd_status st = check_attention(ctx, kv, layer, position, q_heads);
  if (st != ND_OK) return st;
  if (!q || !out || (reinterpret_cast<uintptr_t>(q) & 15))
    return nd_fail(ctx, ND_ERR_INVALID, "q must be a 16-byte aligned device pointer");
  if (q_heads > kStaticAttnQHeads)
    return nd_fail(ctx, ND_ERR_INVALID,
                   "nd_attention_static_d: %u query heads exceed its fixed scratch (at most %u "
                   "query heads; nd_attention_d has no such limit)",
                   q_heads, kStaticAttnQHeads);
  void* scratch = nd_attention_scratch(ctx->device);
  if (!scratch)
    return nd_fail(ctx, ND_ERR_BACKEND, "fixed attention scratch is not set up on device %d",
                   ctx->device);
  const nd_visible vis = nd_kv_visible(kv, position);
  const size_t need =
      (size_t)q_heads * nd_attention_chunks(vis.count, kv->kv_heads) * (kv->head_dim + 2);
  if (need > kStaticAttnPartialWords)
    return nd_fail(ctx, ND_ERR_INVALID,
                   "nd_attention_static_d: %zu partial floats exceed its fixed scratch of %zu",
                   need, kStaticAttnPartialWords);
  float* partials = reinterpret_cast<float*>(scratch);
  uint32_t* counters = reinterpret_cast<uint32_t*>(scratch) + kStaticAttnPartialWords;
  ND_HIP(ctx, nd_launch_attention(kv, layer, position, q, q_heads, out, partials, counters,
                                  nd_pick_stream(ctx, stream)));
  return ND_OK;
}

nd_status nd_attention(nd_ctx* ctx, const nd_kv* kv, uint32_t layer, uint32_t position,
                       const float* q, uint32_t q_heads, float* out) {
  if (!ctx) return nd_fail(nullptr, ND_ERR_BACKEND, "context is NULL");
  nd_status st = check_attention(ctx, kv, layer, position, q_heads);
  if (st != ND_OK) return st;
  if (!q || !out) return nd_fail(ctx, ND_ERR_INVALID, "q or out is NULL");
  const nd_visible vis = nd_kv_visible(kv, position);
  st = ensure_partials(ctx, nd_attention_partial_floats(q_heads, kv->kv_heads, vis.count));
  if (st != ND_OK) return st;
  const size_t bytes = (size_t)q_heads * kv->head_dim * sizeof(float);
  st = ensure_stage(ctx, 2 * align256(bytes));
  if (st != ND_OK) return st;
  float* dq = reinterpret_cast<float*>(ctx->stage);
  float* dout = reinterpret_cast<float*>(reinterpret_cast<char*>(ctx->stage) + align256(bytes));
  ND_HIP(ctx, hipMemcpyAsync(dq, q, bytes, hipMemcpyHostToDevice, ctx->stream));
  ND_HIP(ctx, nd_launch_attention(kv, layer, position, dq, q_heads, dout, ctx->attn_partials,
                                  ctx->attn_counters, ctx->stream));
  ND_HIP(ctx, hipMemcpyAsync(out, dout, bytes, hipMemcpyDeviceToHost, ctx->stream));
  ND_HIP(ctx, hipStreamSynchronize(ctx->stream));
  return ND_OK;
}

// -------------------------------------------------------------- selection

nd_status nd_select(nd_ctx* ctx, const float* logits, uint32_t vocab, const uint32_t* allowed,
                    uint32_t count, uint32_t* id, double* logprob) {
  if (!ctx) return nd_fail(nullptr, ND_ERR_BACKEND, "context is NULL");
  if (!logits || !id || !logprob || vocab == 0)
    return nd_fail(ctx, ND_ERR_INVALID, "nd_select: NULL argument or empty vocabulary");
  if (allowed) {
    if (count == 0) return nd_fail(ctx, ND_ERR_INVALID, "Allowed token set is empty");
    for (uint32_t i = 0; i < count; ++i)
      if (allowed[i] >= vocab)
        return nd_fail(ctx, ND_ERR_INVALID, "Token %u is outside logits", allowed[i]);
  }
  const size_t lb = (size_t)vocab * 4, ab = allowed ? (size_t)count * 4 : 0;
  nd_status st = ensure_stage(ctx, align256(lb) + align256(ab) + 256);
  if (st != ND_OK) return st;
  char* base = reinterpret_cast<char*>(ctx->stage);
  float* dl = reinterpret_cast<float*>(base);
  uint32_t* da = allowed ? reinterpret_cast<uint32_t*>(base + align256(lb)) : nullptr;
  char* res = base + align256(lb) + align256(ab);
  double* dlp = reinterpret_cast<double*>(res);
  uint32_t* did = reinterpret_cast<uint32_t*>(res + 8);
  ND_HIP(ctx, hipMemcpyAsync(dl, logits, lb, hipMemcpyHostToDevice, ctx->stream));
  if (allowed) ND_HIP(ctx, hipMemcpyAsync(da, allowed, ab, hipMemcpyHostToDevice, ctx->stream));
  ND_HIP(ctx, nd_launch_select_list(dl, vocab, da, count, did, dlp, ctx->stream));
  ND_HIP(ctx, hipMemcpyAsync(logprob, dlp, 8, hipMemcpyDeviceToHost, ctx->stream));
  ND_HIP(ctx, hipMemcpyAsync(id, did, 4, hipMemcpyDeviceToHost, ctx->stream));
  ND_HIP(ctx, hipStreamSynchronize(ctx->stream));
  return ND_OK;
}

nd_status nd_select_mask_d(nd_ctx* ctx, const float* logits, uint32_t batch, uint32_t vocab,
                           const uint32_t* mask, uint32_t* ids, double* logprobs, void* stream) {
  if (!ctx) return nd_fail(nullptr, ND_ERR_BACKEND, "context is NULL");
  if (batch && (!logits || !ids || !logprobs || vocab == 0))
    return nd_fail(ctx, ND_ERR_INVALID, "nd_select_mask_d: NULL argument or empty vocabulary");
  if (batch == 0) return ND_OK;
  // Split-selection records and counters: grown (after every stream of the
  // device has drained, as earlier calls may have used any) and zeroed here.
  const size_t need = nd_select_split_bytes(batch);
  if (ctx->sel_split_bytes < need) {
    ND_HIP(ctx, hipDeviceSynchronize());
    if (ctx->sel_split) ND_HIP(ctx, hipFree(ctx->sel_split));
    ctx->sel_split = nullptr;
    ctx->sel_split_bytes = 0;
    ND_HIP(ctx, hipMalloc(&ctx->sel_split, need));
    ND_HIP(ctx, hipMemset(ctx->sel_split, 0, need));
    ND_HIP(ctx, hipDeviceSynchronize());
    ctx->sel_split_bytes = need;
  }
  ND_HIP(ctx, nd_launch_select_mask(logits, batch, vocab, mask, ids, logprobs,
                                    nd_pick_stream(ctx, stream), ctx->sel_split));
  return ND_OK;
}

}  // extern "C"
