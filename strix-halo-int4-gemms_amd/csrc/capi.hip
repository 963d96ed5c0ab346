// C ABI of the gfx950 quantized GEMM library: kernel table, argument
// validation, launch geometry and error reporting.  Declarations and the
// reference interface each symbol replaces are in include/strix_halo_gfx950.h.
#include <cstdio>
#include <cstring>
#include <mutex>
#include <string>
#include <vector>

#include "shk_quant.h"
#include "shk_table.h"

namespace shk {

// Resident workgroups of a persistent launch, cached per (kernel, device):
// the occupancy query walks the kernel's resource use on the host.
hipError_t persistent_grid(const void* kernel, int block, unsigned tiles, unsigned* grid) {
  struct Slot {
    const void* kernel;
    int device, block;
    unsigned slots;
  };
  static std::mutex lock;
  static std::vector<Slot> cache;
  int dev = 0;
  hipError_t err = hipGetDevice(&dev);
  if (err != hipSuccess) return err;
  unsigned slots = 0;
  {
    std::lock_guard<std::mutex> g(lock);
    for (const Slot& c : cache)
      if (c.kernel == kernel && c.device == dev && c.block == block) slots = c.slots;
  }
  if (slots == 0) {
    int cus = 0, occ = 0;
    err = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
    if (err == hipSuccess) err = hipOccupancyMaxActiveBlocksPerMultiprocessor(&occ, kernel, block, 0);
    if (err != hipSuccess) return err;
    slots = (unsigned)(cus > 0 ? cus : 1) * (unsigned)(occ > 0 ? occ : 1);
    if (slots >= 8) slots &= ~7u;  // a workgroup keeps its XCD across its tiles
    std::lock_guard<std::mutex> g(lock);
    cache.push_back(Slot{kernel, dev, block, slots});
  }
  *grid = slots < tiles ? slots : tiles;
  return hipSuccess;
}

// Clears n16 16-byte units at p: the arrival counters of a split skinny
// launch on the no-allocation path, whose scratch the fp6 conversions of
// other calls may have left dirty.  A kernel, not a memset, so that a graph
// capture records an ordinary kernel node.
__global__ __launch_bounds__(256) void clear_counters_kernel(int4* p, unsigned n16) {
  const unsigned i = blockIdx.x * 256u + threadIdx.x;
  if (i < n16) p[i] = make_int4(0, 0, 0, 0);
}

}  // namespace shk

namespace {

using shk::Entry;

thread_local std::string g_last_error;

int fail(const std::string& msg) {
  g_last_error = msg;
  return 1;
}

int fail_hip(const char* what, hipError_t err) {
  // Clear the sticky error so the next call starts clean (dispatch.cpp:150-156).
  (void)hipGetLastError();
  return fail(std::string(what) + " failed: " + hipGetErrorString(err));
}

const std::vector<Entry>& table() {
  static const std::vector<Entry> t = [] {
    std::vector<Entry> v;
    shk::append_dense_f6(v, SHK_LAYOUT_NN);
    shk::append_dense_dma_4_0(v);
    shk::append_dense_4_0(v);
    shk::append_dense_f6(v, SHK_LAYOUT_NT);
    shk::append_dense_dma_4_1(v);
    shk::append_dense_4_1(v);
    shk::append_dense_f6(v, SHK_LAYOUT_TN);
    shk::append_dense_dma_4_2(v);
    shk::append_dense_4_2(v);
    shk::append_dense_dma_8_0(v);
    shk::append_dense_8_0(v);
    shk::append_dense_dma_8_1(v);
    shk::append_dense_8_1(v);
    shk::append_dense_dma_8_2(v);
    shk::append_dense_8_2(v);
    shk::append_ragged_0(v);
    shk::append_ragged_1(v);
    shk::append_ragged_2(v);
    shk::append_ragged_3(v);
    shk::append_persistent_f6(v, SHK_LAYOUT_NN);
    shk::append_persistent_4_0(v);
    shk::append_persistent_f6(v, SHK_LAYOUT_NT);
    shk::append_persistent_4_1(v);
    shk::append_persistent_f6(v, SHK_LAYOUT_TN);
    shk::append_persistent_4_2(v);
    shk::append_split_4_0(v);
    shk::append_split_4_1(v);
    shk::append_split_4_2(v);
    shk::append_split_8_0(v);
    shk::append_split_8_1(v);
    shk::append_split_8_2(v);
    shk::append_skinny_4_0(v);
    shk::append_skinny_4_1(v);
    shk::append_skinny_4_2(v);
    shk::append_skinny_8_0(v);
    shk::append_skinny_8_1(v);
    shk::append_skinny_8_2(v);
    for (size_t i = 0; i < v.size(); ++i) v[i].d.index = (int32_t)i;
    return v;
  }();
  return t;
}

// Makes `device` current for the duration of a launch and restores the
// caller's device afterwards.
class DeviceGuard {
 public:
  explicit DeviceGuard(int device) {
    if (hipGetDevice(&prev_) != hipSuccess) prev_ = -1;
    if (prev_ != device) {
      err_ = hipSetDevice(device);
      switched_ = err_ == hipSuccess;
    }
  }
  ~DeviceGuard() {
    if (switched_ && prev_ >= 0) (void)hipSetDevice(prev_);
  }
  hipError_t error() const { return err_; }

 private:
  int prev_ = -1;
  bool switched_ = false;
  hipError_t err_ = hipSuccess;
};

bool aligned(const void* p, uintptr_t a) { return (reinterpret_cast<uintptr_t>(p) % a) == 0; }

}  // namespace

// Scratch of amd_strix_halo_kernels_launch_gemm_noalloc: the fp6 operand
// workspace of callers that cannot allocate device memory.  Each device the
// library runs on holds its own copy from the code object's load until the
// process ends.  In host code `scratch` names a host-side stand-in, never the
// device array: kernels and copies get the per-device address from
// scratch_address() instead.
static __device__ __align__(256) uint8_t scratch[SHK_NOALLOC_SCRATCH_BYTES];

namespace {

// Device address of `scratch` on the current device (`device`), looked up
// once per device with hipGetSymbolAddress and cached.
int scratch_address(int device, void** ptr) {
  constexpr int kMaxDevices = 64;
  static std::mutex lock;
  static void* cache[kMaxDevices] = {};
  if (device < 0 || device >= kMaxDevices)
    return fail("device index " + std::to_string(device) + " is out of range for the scratch table");
  std::lock_guard<std::mutex> g(lock);
  if (cache[device] == nullptr) {
    void* p = nullptr;
    const hipError_t err = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (err != hipSuccess) return fail_hip("hipGetSymbolAddress(scratch)", err);
    if (p == nullptr || !aligned(p, 256)) return fail("the scratch array has no usable device address");
    cache[device] = p;
  }
  *ptr = cache[device];
  return 0;
}

int lookup(int index, int family, const Entry** out) {
  const auto& t = table();
  if (index < 0 || index >= (int)t.size()) {
    return fail("kernel index " + std::to_string(index) + " is out of range [0, " + std::to_string(t.size()) +
                ")");
  }
  if (t[index].d.family != family) {
    return fail("kernel index " + std::to_string(index) + " belongs to another kernel family");
  }
  *out = &t[index];
  return 0;
}

// Subchannel size check shared by the three families.
int check_subchannel(const shk_kernel_desc& d, int subchannel) {
  if (d.scale_mode == SHK_SCALE_PER_CHANNEL) {
    if (subchannel != 0) return fail("per-channel kernels take subchannel = 0");
    return 0;
  }
  const bool pow2 = subchannel > 0 && (subchannel & (subchannel - 1)) == 0;
  if (!pow2 || subchannel < d.min_subchannel || subchannel > d.max_subchannel) {
    return fail("subchannel size " + std::to_string(subchannel) + " is not served by this kernel (supports " +
                std::to_string(d.min_subchannel) + ".." + std::to_string(d.max_subchannel) + ")");
  }
  return 0;
}

int check_out_mode(int out_mode) {
  if (out_mode != SHK_OUT_BF16 && out_mode != SHK_OUT_F32 && out_mode != SHK_OUT_I32)
    return fail("unknown output mode " + std::to_string(out_mode));
  return 0;
}

// Workspace of a dense entry: both operands in fp6 block format for FP6
// entries (and for per-channel calls with K > F6_MAX_K, the [m, b_cols]
// int32 sums of their K slices past the operands); for STREAM entries the
// arrival counters and exact partials of a split K (shk::sk_workspace_bytes);
// nothing otherwise.
uint64_t dense_workspace_bytes(const shk_kernel_desc& d, int32_t m, int32_t n, int32_t k) {
  if (d.operand_format == SHK_OPERANDS_STREAM) return shk::sk_workspace_bytes(d, m, n, k);
  if (d.operand_format != SHK_OPERANDS_FP6) return 0;
  const long b_cols = d.epilogue_kind == SHK_EPI_KIND_SWIGLU ? 2L * n : (long)n;
  uint64_t bytes = shk::f6_operand_bytes(m, k) + shk::f6_operand_bytes(b_cols, k);
  if (d.scale_mode == SHK_SCALE_PER_CHANNEL && k > shk::F6_MAX_K) bytes += 4ull * (uint64_t)m * (uint64_t)b_cols;
  return bytes;
}

// Largest K for which the x16-widened int4 products of one int32 accumulator
// cannot overflow: |sum| <= 128 * 128 * K < 2^31, so K < 131072 (at K =
// 131072 a row and column of -8 sum to exactly 2^31).  A split-K entry's
// accumulator holds one slice of K / split values.
constexpr int kMaxInt4AccK = 131071;

// Largest K a dense entry runs: fp6 entries up to F6_MAX_K_SLICED, except
// the persistent per-channel tile, which multiplies whole K in one pass
// (F6_MAX_K); int4 per-channel STREAM entries F6_MAX_K_SLICED as well (their
// x256 int32 sums stay within 1023 stages per wave through the split count);
// int4 per-channel entries of the int8 engines kMaxInt4AccK per K slice; no
// bound otherwise.
long dense_max_k(const shk_kernel_desc& d) {
  if (d.operand_format == SHK_OPERANDS_STREAM)
    return (d.dtype_bits == 4 && d.scale_mode == SHK_SCALE_PER_CHANNEL) ? shk::F6_MAX_K_SLICED : 0x7FFFFFFFL;
  if (d.operand_format == SHK_OPERANDS_FP6)
    return (d.scale_mode == SHK_SCALE_PER_CHANNEL && d.schedule == SHK_SCHEDULE_PERSISTENT) ? shk::F6_MAX_K
                                                                                            : shk::F6_MAX_K_SLICED;
  if (d.dtype_bits == 4 && d.scale_mode == SHK_SCALE_PER_CHANNEL)
    return (long)kMaxInt4AccK * (d.split_k > 1 ? d.split_k : 1);
  return 0x7FFFFFFFL;
}

// Workspace argument of prepare_dense for a call that runs in the library's
// scratch array: validated against the array's size; the caller sets the
// workspace pointer (p.work) to the array's device address afterwards.
void* const kScratchPending = reinterpret_cast<void*>(static_cast<uintptr_t>(256));

// A validated dense call.  PHASE_ALL is a whole launch; the other phases are
// the separately launched parts of a fp6 entry: converting A, converting B,
// and the GEMM on converted operands.  Each phase checks the arguments it
// uses; all of them check the shape and the workspace.
enum Phase { PHASE_ALL, PHASE_CONVERT_A, PHASE_CONVERT_B, PHASE_GEMM };

struct DenseCall {
  const Entry* e = nullptr;
  shk::DenseArgs p{};
  long tiles = 0;
};

int prepare_dense(DenseCall& c, int kernel_index, Phase phase, const void* a, const void* b, const void* a_scale,
                  const void* b_scale, void* out, int32_t m, int32_t n, int32_t k, int32_t subchannel,
                  int32_t epilogue, int32_t out_mode, void* workspace, uint64_t workspace_bytes) {
  if (lookup(kernel_index, SHK_FAMILY_DENSE, &c.e)) return 1;
  const shk_kernel_desc& d = c.e->d;
  const bool fp6 = d.operand_format == SHK_OPERANDS_FP6;
  const bool stream = d.operand_format == SHK_OPERANDS_STREAM;
  const bool uses_a = phase == PHASE_ALL || phase == PHASE_CONVERT_A;
  const bool uses_b = phase == PHASE_ALL || phase == PHASE_CONVERT_B;
  const bool gemm = phase == PHASE_ALL || phase == PHASE_GEMM;
  if (phase != PHASE_ALL && !fp6)
    return fail("kernel " + std::to_string(kernel_index) +
                " reads its operands directly; only fp6 entries convert them separately");
  if ((uses_a && a == nullptr) || (uses_b && b == nullptr) ||
      (gemm && (a_scale == nullptr || b_scale == nullptr || out == nullptr))) {
    if (phase == PHASE_ALL) return fail("a, b, a_scale, b_scale, and out pointers must be non-null");
    if (phase == PHASE_GEMM) return fail("a_scale, b_scale, and out pointers must be non-null");
    return fail("the operand pointer must be non-null");
  }
  if (m <= 0 || n <= 0 || k <= 0)
    return fail("M, N, and K must be positive; got (" + std::to_string(m) + ", " + std::to_string(n) + ", " +
                std::to_string(k) + ")");
  std::string why;
  if (m % d.block_m) why += "M=" + std::to_string(m) + " is not divisible by BLOCK_M=" + std::to_string(d.block_m);
  if (n % d.block_n) {
    if (!why.empty()) why += "; ";
    why += "N=" + std::to_string(n) + " is not divisible by BLOCK_N=" + std::to_string(d.block_n);
  }
  const int split = d.split_k > 1 ? d.split_k : 1;
  if (k % (d.block_k * split)) {
    if (!why.empty()) why += "; ";
    why += "K=" + std::to_string(k) + " is not divisible by BLOCK_K*SPLIT_K=" + std::to_string(d.block_k * split);
  }
  if (d.scale_mode == SHK_SCALE_SUBCHANNEL && subchannel > 0 && k % subchannel) {
    if (!why.empty()) why += "; ";
    why += "K=" + std::to_string(k) + " is not divisible by SUBCHANNEL=" + std::to_string(subchannel);
  }
  if (split > 1 && !stream && d.scale_mode == SHK_SCALE_SUBCHANNEL && subchannel > 0 && (k / split) % subchannel) {
    if (!why.empty()) why += "; ";
    why += "K/SPLIT_K=" + std::to_string(k / split) + " is not divisible by SUBCHANNEL=" + std::to_string(subchannel);
  }
  if (!why.empty()) return fail("kernel " + std::to_string(kernel_index) + " requires tile-multiple shape: " + why);
  if (split > 1 && gemm && epilogue != SHK_EPILOGUE_NONE)
    return fail("split-K kernels support the NONE epilogue only (SPLIT_K=" + std::to_string(split) + ")");
  if (split > 1 && gemm && out_mode != SHK_OUT_F32)
    return fail("split-K kernels write float32 output (out_mode " + std::to_string(SHK_OUT_F32) + ")");
  const bool swiglu = d.epilogue_kind == SHK_EPI_KIND_SWIGLU;
  if (gemm) {
    if (check_subchannel(d, subchannel)) return 1;
    if (check_out_mode(out_mode)) return 1;
    if (swiglu ? epilogue != SHK_EPILOGUE_SWIGLU : (epilogue != SHK_EPILOGUE_NONE && epilogue != SHK_EPILOGUE_RELU2))
      return fail("epilogue " + std::to_string(epilogue) + " does not match the kernel's epilogue kind");
  }
  if (k > dense_max_k(d)) {
    if (fp6 || stream) return fail("kernel " + std::to_string(kernel_index) + " supports K <= " +
                                   std::to_string(dense_max_k(d)) + "; got " + std::to_string(k));
    return fail("int4 per-channel kernels support K <= " + std::to_string(kMaxInt4AccK) +
                (split > 1 ? " per K slice (K/SPLIT_K); got K/SPLIT_K=" + std::to_string(k / split)
                           : "; got " + std::to_string(k)));
  }
  if (fp6 && workspace == kScratchPending) {
    // the no-allocation entry point: the library's scratch array, whose
    // device address the caller fills in after validation
    const uint64_t need = dense_workspace_bytes(d, m, n, k);
    if (need > workspace_bytes)
      return fail("kernel " + std::to_string(kernel_index) + " needs " + std::to_string(need) +
                  " bytes of scratch for this shape; the no-allocation entry point's scratch holds at most " +
                  std::to_string(workspace_bytes) + " bytes (use amd_strix_halo_kernels_launch_gemm_ws)");
  } else if (fp6) {
    const uint64_t need = dense_workspace_bytes(d, m, n, k);
    if (workspace == nullptr || workspace_bytes < need)
      return fail("kernel " + std::to_string(kernel_index) + " converts its operands into a workspace of " +
                  std::to_string(need) + " bytes (amd_strix_halo_kernels_gemm_workspace_bytes)");
    if (!aligned(workspace, 16)) return fail("the workspace must be 16-byte aligned");
  }
  if (stream && gemm) {
    // K split over workgroups only with a (zeroed-counter) workspace
    const bool with_ws = workspace != nullptr;
    const uint64_t need = dense_workspace_bytes(d, m, n, k);
    if (with_ws && workspace != kScratchPending) {
      if (workspace_bytes < need)
        return fail("kernel " + std::to_string(kernel_index) + " needs a workspace of " + std::to_string(need) +
                    " bytes for this shape (amd_strix_halo_kernels_gemm_workspace_bytes)");
      if (need > 0 && !aligned(workspace, 16)) return fail("the workspace must be 16-byte aligned");
    } else if (with_ws && need > workspace_bytes) {
      return fail("kernel " + std::to_string(kernel_index) + " needs " + std::to_string(need) +
                  " bytes of scratch for this shape; the no-allocation entry point's scratch holds at most " +
                  std::to_string(workspace_bytes) + " bytes (use amd_strix_halo_kernels_launch_gemm_ws)");
    }
    const int splits = shk::sk_split_count(d, m, n, k, with_ws && need > 0);
    if (splits == 0)
      return fail("kernel " + std::to_string(kernel_index) + " splits K=" + std::to_string(k) +
                  " over workgroups, which needs a workspace (amd_strix_halo_kernels_launch_gemm_ws)");
    c.p.sk_splits = splits;
  }
  if (gemm && (!aligned(out, 16) || !aligned(b_scale, 8) || !aligned(a_scale, 2)))
    return fail("out must be 16-byte aligned and b_scale 8-byte aligned");

  const long kbytes = (long)k * d.dtype_bits / 8;
  const int b_cols = swiglu ? 2 * n : n;
  shk::DenseArgs& p = c.p;
  p.a = static_cast<const uint8_t*>(a);
  p.b = static_cast<const uint8_t*>(b);
  p.a_scale = static_cast<const uint16_t*>(a_scale);
  p.b_scale = static_cast<const uint16_t*>(b_scale);
  p.out = out;
  p.M = m;
  p.N = n;
  p.K = k;
  const bool a_km = d.layout != SHK_LAYOUT_TN;
  const bool b_km = d.layout == SHK_LAYOUT_NT;
  p.lda = a_km ? kbytes : m;
  p.ldb = b_km ? kbytes : b_cols;
  p.b_cols = b_cols;
  p.subchannel = subchannel;
  p.scale_cols = subchannel > 0 ? (k + subchannel - 1) / subchannel : 1;
  p.epilogue = epilogue == SHK_EPILOGUE_RELU2 ? shk::EPI_RELU2 : shk::EPI_NONE;
  p.out_mode = out_mode;
  // 16-byte pieces for K-major operands and for every operand of the
  // direct-to-LDS and fp6 tiles; 8-byte rows otherwise.
  const bool dma = d.num_stages > 2 || fp6 || stream;
  const int a_need = (a_km || dma) ? 16 : 8;
  const int b_need = (b_km || dma) ? 16 : 8;
  p.a_aligned = !uses_a || (aligned(a, a_need) && p.lda % a_need == 0);
  p.b_aligned = !uses_b || (aligned(b, b_need) && p.ldb % b_need == 0);
  p.group_m = d.group_size_m;
  p.layout = d.layout;
  p.work = static_cast<uint8_t*>(workspace);
  if (stream && p.sk_splits <= 1) p.work = nullptr;
  // Operands are addressed with 32-bit buffer offsets.
  if ((unsigned long long)kbytes * (unsigned long long)m >= (1ull << 32) ||
      (unsigned long long)kbytes * (unsigned long long)b_cols >= (1ull << 32))
    return fail("dense operands must each be smaller than 4 GiB");
  // Output stores address a tile's rows with 32-bit offsets from its first
  // element: 256 rows of fp32 (or int32 [up | gate]) must stay below 4 GiB.
  if ((unsigned long long)b_cols * 4ull * 256ull >= (1ull << 32))
    return fail("dense output rows are limited to 4194304 bytes");
  if (!p.a_aligned || !p.b_aligned)
    return fail("kernel " + std::to_string(kernel_index) + " needs " + std::to_string(a_need) +
                "-byte aligned A and " + std::to_string(b_need) + "-byte aligned B data pointers");
  c.tiles = (long)(m / d.block_m) * (n / d.block_n);
  if (c.tiles > 0x7FFFFFFFL) return fail("too many output tiles");
  return 0;
}


// Workspace of a ragged entry: both operands in fp6 block format for FP6
// entries (forward: A, then B per group; backward: A per group, then B per
// group), nothing otherwise.
uint64_t ragged_workspace_bytes(const shk_kernel_desc& d, int32_t m, int32_t n, int32_t k_packed, int32_t groups) {
  if (d.operand_format != SHK_OPERANDS_FP6) return 0;
  if (d.family == SHK_FAMILY_RAGGED_FWD)
    return shk::f6_ragged_fwd_workspace(m, n, 2 * k_packed, groups, d.scale_mode == SHK_SCALE_SUBCHANNEL);
  return shk::f6_ragged_bwd_workspace(m, n, 2 * k_packed, groups, d.scale_mode == SHK_SCALE_SUBCHANNEL);
}

// Requirements of the fp6 ragged entries: a K that keeps fp32 sums exact,
// whole 16-byte output units (N a multiple of 8, out 16-byte aligned) and
// 4-scale loads (b_scale 8-byte aligned), 32-bit offsets within a tile, and
// a large enough workspace.  Operands may have any alignment.
int check_f6_ragged(const shk_kernel_desc& d, int32_t subchannel, const void* b_scale, const void* out, int32_t m,
                    int32_t n, int32_t k_packed, int32_t groups, const void* workspace, uint64_t workspace_bytes) {
  const int k = 2 * k_packed;
  if (k > shk::F6_MAX_K) return fail("fp6 kernels support K <= " + std::to_string(shk::F6_MAX_K));
  const bool sub = d.scale_mode == SHK_SCALE_SUBCHANNEL;
  // the tile reads a_scale [M, ceil(K/S)] in whole dwords, which covers the
  // last value only when M * ceil(K/S) is even
  const int scale_cols = sub ? (k + subchannel - 1) / subchannel : 1;
  if (sub && (long long)m * scale_cols % 2)
    return fail("kernel " + std::to_string(d.index) + " needs M * ceil(K/subchannel) to be even; got M=" +
                std::to_string(m) + ", ceil(K/subchannel)=" + std::to_string(scale_cols));
  // groups of 32 take their a_scale values in pairs, one dword per row
  if (sub && subchannel == 32 && scale_cols % 2)
    return fail("kernel " + std::to_string(d.index) + " needs ceil(K/32) to be even with subchannel 32; got " +
                std::to_string(scale_cols));
  if (n % 8) return fail("kernel " + std::to_string(d.index) + " needs N to be a multiple of 8; got " + std::to_string(n));
  if (!aligned(out, 16) || !aligned(b_scale, 8)) return fail("out must be 16-byte aligned and b_scale 8-byte aligned");
  if ((unsigned long long)n * 4ull * 256ull >= (1ull << 32)) return fail("ragged output rows are limited to 4194304 bytes");
  // nothing runs without rows, columns or groups
  const uint64_t need = (m == 0 || n == 0 || groups == 0) ? 0 : ragged_workspace_bytes(d, m, n, k_packed, groups);
  if (need > 0 && (workspace == nullptr || workspace_bytes < need))
    return fail("kernel " + std::to_string(d.index) + " converts its operands into a workspace of " +
                std::to_string(need) + " bytes (amd_strix_halo_kernels_ragged_workspace_bytes)");
  if (need > 0 && !aligned(workspace, 16)) return fail("the workspace must be 16-byte aligned");
  return 0;
}

}  // namespace

extern "C" {

int amd_strix_halo_kernels_dispatch_version(void) { return 2; }

int amd_strix_halo_kernels_has_compiled_code_objects(void) { return 1; }

int amd_strix_halo_kernels_has_hip_runtime(void) {
  int n = 0;
  if (hipGetDeviceCount(&n) != hipSuccess) {
    (void)hipGetLastError();
    return 0;
  }
  return n > 0 ? 1 : 0;
}

int amd_strix_halo_kernels_has_linked_kernels(void) {
  int n = 0;
  if (hipGetDeviceCount(&n) != hipSuccess) {
    (void)hipGetLastError();
    return 0;
  }
  for (int i = 0; i < n; ++i) {
    hipDeviceProp_t prop;
    if (hipGetDeviceProperties(&prop, i) != hipSuccess) {
      (void)hipGetLastError();
      continue;
    }
    if (std::strncmp(prop.gcnArchName, "gfx950", 6) == 0) return 1;
  }
  return 0;
}

const char* amd_strix_halo_kernels_last_error(void) { return g_last_error.c_str(); }

const char* amd_strix_halo_kernels_arch(void) { return "gfx950"; }

int amd_strix_halo_kernels_kernel_table_size(void) { return (int)table().size(); }

int amd_strix_halo_kernels_kernel_table_entry(int index, shk_kernel_desc* out) {
  g_last_error.clear();
  if (out == nullptr) return fail("out must be non-null");
  const auto& t = table();
  if (index < 0 || index >= (int)t.size()) return fail("kernel index out of range");
  *out = t[index].d;
  return 0;
}

namespace {

// Throughput measured on MI355X for the entries the benchmark configurations
// time (the Python registry's kernel_table.measured_tops): the first
// ranking key of a selection, before the tile area.
double measured_score(const shk_kernel_desc& d, int m) {
  if (d.schedule != SHK_SCHEDULE_STANDARD || d.split_k > 1) return 0.0;
  if (d.operand_format == SHK_OPERANDS_FP6) {
    if (d.scale_mode == SHK_SCALE_SUBCHANNEL) return 2001.0;
    return d.epilogue_kind == SHK_EPI_KIND_PLAIN ? 3504.0 : 3161.0;
  }
  if (d.operand_format == SHK_OPERANDS_STREAM) {  // the skinny tiles (subchannel: by tile height, up to 256 rows)
    if (d.scale_mode == SHK_SCALE_PER_CHANNEL) return 241.0;
    if (m > 256) return 0.0;
    return d.block_m == 16 ? 96.0 : (d.block_m == 32 ? 184.0 : 152.0);
  }
  if (d.dtype_bits == 8 && d.num_stages == 4 && d.block_m == 256)
    return d.epilogue_kind == SHK_EPI_KIND_SWIGLU ? 2014.0 : 2270.0;
  return 0.0;
}

// Whether a dense entry serves the request's family: SwiGLU entries serve
// SwiGLU, persistent and split-K entries the plain epilogue, the others
// plain and ReLU2; subchannel entries a group size within their range.
bool serves_family(const shk_kernel_desc& d, int bits, int layout, int subchannel, int epilogue, int schedule,
                   int split_k) {
  if (d.family != SHK_FAMILY_DENSE || d.dtype_bits != bits || d.layout != layout || d.schedule != schedule)
    return false;
  const int s = d.split_k > 1 ? d.split_k : 1;
  if (split_k > 0 && s != split_k) return false;
  if (subchannel == 0 ? d.scale_mode != SHK_SCALE_PER_CHANNEL
                      : (d.scale_mode != SHK_SCALE_SUBCHANNEL || subchannel < d.min_subchannel ||
                         subchannel > d.max_subchannel))
    return false;
  if (d.epilogue_kind == SHK_EPI_KIND_SWIGLU) return epilogue == SHK_EPILOGUE_SWIGLU;
  if (d.schedule == SHK_SCHEDULE_PERSISTENT || s > 1) return epilogue == SHK_EPILOGUE_NONE;
  return epilogue == SHK_EPILOGUE_NONE || epilogue == SHK_EPILOGUE_RELU2;
}

// The launch-shape rule of prepare_dense, without side effects.
bool accepts_shape(const shk_kernel_desc& d, int m, int n, int k, int subchannel) {
  const int s = d.split_k > 1 ? d.split_k : 1;
  if (m % d.block_m || n % d.block_n || k % (d.block_k * s)) return false;
  if (subchannel > 0 && k % subchannel) return false;
  if (subchannel > 0 && s > 1 && d.operand_format != SHK_OPERANDS_STREAM && (k / s) % subchannel) return false;
  return k <= dense_max_k(d);
}

}  // namespace

int amd_strix_halo_kernels_select_dense(int32_t dtype_bits, int32_t layout, int32_t subchannel, int32_t epilogue,
                                        int32_t schedule, int32_t split_k, int32_t m, int32_t n, int32_t k,
                                        int32_t* kernel_index) {
  g_last_error.clear();
  if (kernel_index == nullptr) return fail("kernel_index must be non-null");
  if (dtype_bits != 4 && dtype_bits != 8) return fail("dtype_bits must be 4 or 8");
  if (layout < SHK_LAYOUT_NN || layout > SHK_LAYOUT_TT) return fail("layout must be 0 (NN), 1 (NT), 2 (TN) or 3 (TT)");
  if (subchannel != 0 && subchannel != 32 && subchannel != 64 && subchannel != 128 && subchannel != 256)
    return fail("subchannel must be 0 (per-channel) or one of 32, 64, 128, 256");
  if (epilogue < SHK_EPILOGUE_NONE || epilogue > SHK_EPILOGUE_SWIGLU) return fail("epilogue must be 0, 1 or 2");
  if (schedule != SHK_SCHEDULE_STANDARD && schedule != SHK_SCHEDULE_PERSISTENT)
    return fail("schedule must be 0 (standard) or 1 (persistent)");
  if (split_k < 0) return fail("split_k must be 0 (any) or positive");
  if (m <= 0 || n <= 0 || k <= 0)
    return fail("M, N, and K must be positive; got (" + std::to_string(m) + ", " + std::to_string(n) + ", " +
                std::to_string(k) + ")");
  const auto& t = table();
  int best = -1;
  double best_score = -1.0;
  long best_area = -1;
  for (int i = 0; i < (int)t.size(); ++i) {
    const shk_kernel_desc& d = t[i].d;
    if (!serves_family(d, dtype_bits, layout, subchannel, epilogue, schedule, split_k)) continue;
    if (!accepts_shape(d, m, n, k, subchannel)) continue;
    const double score = measured_score(d, m);
    const long area = (long)d.block_m * d.block_n;
    if (score > best_score || (score == best_score && area > best_area)) {
      best = i;
      best_score = score;
      best_area = area;
    }
  }
  if (best < 0)
    return fail("no kernel for dtype_bits=" + std::to_string(dtype_bits) + ", subchannel=" +
                std::to_string(subchannel) + ", epilogue=" + std::to_string(epilogue) + ", layout=" +
                std::to_string(layout) + ", schedule=" + std::to_string(schedule) + ", split_k=" +
                std::to_string(split_k) + ", shape=(" + std::to_string(m) + ", " + std::to_string(n) + ", " +
                std::to_string(k) + ")");
  *kernel_index = best;
  return 0;
}

int amd_strix_halo_kernels_gemm_workspace_bytes(int kernel_index, int32_t m, int32_t n, int32_t k,
                                                uint64_t* bytes) {
  g_last_error.clear();
  if (bytes == nullptr) return fail("bytes must be non-null");
  const Entry* e = nullptr;
  if (lookup(kernel_index, SHK_FAMILY_DENSE, &e)) return 1;
  if (m < 0 || n < 0 || k < 0) return fail("M, N, and K must be non-negative");
  *bytes = dense_workspace_bytes(e->d, m, n, k);
  return 0;
}

int amd_strix_halo_kernels_launch_gemm(int kernel_index, int device_index, uintptr_t stream, const void* a,
                                       const void* b, const void* a_scale, const void* b_scale, void* out,
                                       int32_t m, int32_t n, int32_t k, int32_t subchannel, int32_t epilogue,
                                       int32_t out_mode) {
  return amd_strix_halo_kernels_launch_gemm_ws(kernel_index, device_index, stream, a, b, a_scale, b_scale, out, m,
                                               n, k, subchannel, epilogue, out_mode, nullptr, 0);
}

int amd_strix_halo_kernels_launch_gemm_ws(int kernel_index, int device_index, uintptr_t stream, const void* a,
                                          const void* b, const void* a_scale, const void* b_scale, void* out,
                                          int32_t m, int32_t n, int32_t k, int32_t subchannel, int32_t epilogue,
                                          int32_t out_mode, void* workspace, uint64_t workspace_bytes) {
  g_last_error.clear();
  DenseCall c;
  if (prepare_dense(c, kernel_index, PHASE_ALL, a, b, a_scale, b_scale, out, m, n, k, subchannel, epilogue,
                    out_mode, workspace, workspace_bytes))
    return 1;
  DeviceGuard guard(device_index);
  if (guard.error() != hipSuccess) return fail_hip("hipSetDevice", guard.error());
  const unsigned split = c.e->d.split_k > 1 ? (unsigned)c.e->d.split_k : 1u;
  const hipError_t err = c.e->dense(c.p, dim3((unsigned)c.tiles, split), reinterpret_cast<hipStream_t>(stream));
  if (err != hipSuccess) return fail_hip("kernel launch", err);
  return 0;
}

int amd_strix_halo_kernels_launch_gemm_noalloc(int kernel_index, int device_index, uintptr_t stream, const void* a,
                                               const void* b, const void* a_scale, const void* b_scale, void* out,
                                               int32_t m, int32_t n, int32_t k, int32_t subchannel,
                                               int32_t epilogue, int32_t out_mode) {
  g_last_error.clear();
  DenseCall c;
  if (prepare_dense(c, kernel_index, PHASE_ALL, a, b, a_scale, b_scale, out, m, n, k, subchannel, epilogue,
                    out_mode, kScratchPending, SHK_NOALLOC_SCRATCH_BYTES))
    return 1;
  DeviceGuard guard(device_index);
  if (guard.error() != hipSuccess) return fail_hip("hipSetDevice", guard.error());
  const bool split_stream = c.e->d.operand_format == SHK_OPERANDS_STREAM && c.p.sk_splits > 1;
  if (c.e->d.operand_format == SHK_OPERANDS_FP6 || split_stream) {
    void* ptr = nullptr;
    if (scratch_address(device_index, &ptr)) return 1;
    c.p.work = static_cast<uint8_t*>(ptr);
  } else {
    c.p.work = nullptr;
  }
  const hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  if (split_stream) {
    // the partial slots are written before they are read; only the counters
    // must start at zero (256-byte multiple, below the scratch size)
    const unsigned n16 = (unsigned)(shk::sk_counter_bytes(c.e->d, m, n) / 16);
    hipLaunchKernelGGL(shk::clear_counters_kernel, dim3((n16 + 255) / 256), dim3(256), 0, s,
                       reinterpret_cast<int4*>(c.p.work), n16);
    const hipError_t cerr = hipGetLastError();
    if (cerr != hipSuccess) return fail_hip("kernel launch", cerr);
  }
  const unsigned split = c.e->d.split_k > 1 ? (unsigned)c.e->d.split_k : 1u;
  const hipError_t err = c.e->dense(c.p, dim3((unsigned)c.tiles, split), s);
  if (err != hipSuccess) return fail_hip("kernel launch", err);
  return 0;
}

int amd_strix_halo_kernels_gemm_convert(int kernel_index, int device_index, uintptr_t stream, int32_t operand,
                                        const void* src, int32_t m, int32_t n, int32_t k, void* workspace,
                                        uint64_t workspace_bytes) {
  g_last_error.clear();
  if (operand != 0 && operand != 1) return fail("operand must be 0 (A) or 1 (B)");
  DenseCall c;
  if (prepare_dense(c, kernel_index, operand == 0 ? PHASE_CONVERT_A : PHASE_CONVERT_B, operand == 0 ? src : nullptr,
                    operand == 1 ? src : nullptr, nullptr, nullptr, nullptr, m, n, k, 0, 0, SHK_OUT_BF16, workspace,
                    workspace_bytes))
    return 1;
  DeviceGuard guard(device_index);
  if (guard.error() != hipSuccess) return fail_hip("hipSetDevice", guard.error());
  const hipError_t err = shk::f6_convert_operand(c.p, operand, c.e->d.epilogue_kind == SHK_EPI_KIND_SWIGLU,
                                                 reinterpret_cast<hipStream_t>(stream));
  if (err != hipSuccess) return fail_hip("kernel launch", err);
  return 0;
}

int amd_strix_halo_kernels_launch_gemm_converted(int kernel_index, int device_index, uintptr_t stream,
                                                 const void* a_scale, const void* b_scale, void* out, int32_t m,
                                                 int32_t n, int32_t k, int32_t epilogue, int32_t out_mode,
                                                 const void* workspace, uint64_t workspace_bytes) {
  g_last_error.clear();
  DenseCall c;
  if (prepare_dense(c, kernel_index, PHASE_GEMM, nullptr, nullptr, a_scale, b_scale, out, m, n, k, 0, epilogue,
                    out_mode, const_cast<void*>(workspace), workspace_bytes))
    return 1;
  DeviceGuard guard(device_index);
  if (guard.error() != hipSuccess) return fail_hip("hipSetDevice", guard.error());
  const hipError_t err = c.e->converted(c.p, dim3((unsigned)c.tiles), reinterpret_cast<hipStream_t>(stream));
  if (err != hipSuccess) return fail_hip("kernel launch", err);
  return 0;
}

int32_t amd_strix_halo_kernels_ragged_task_capacity(int32_t rows, int32_t groups, int32_t tile,
                                                    int32_t align_tile) {
  if (rows < 0 || groups < 0 || tile <= 0 || align_tile <= 0) return 0;
  (void)align_tile;  // align_tile <= tile bounds every group's extra block by one
  const long cap = (long)rows / tile + 2L * groups + 1;
  return cap > 0x7FFFFFFFL ? 0x7FFFFFFF : (int32_t)cap;
}

int amd_strix_halo_kernels_ragged_group_info(int device_index, uintptr_t stream, const int32_t* group_sizes,
                                             int32_t groups, int32_t tile, int32_t align_tile, int32_t capacity,
                                             int32_t* tasks_i32, int32_t* num_tasks_i32, int64_t* info_i64) {
  g_last_error.clear();
  if (groups < 0) return fail("groups must be non-negative");
  if (groups > shk::max_info_groups())
    return fail("at most " + std::to_string(shk::max_info_groups()) + " groups are supported");
  if (tile <= 0) return fail("tile must be positive");
  if (align_tile <= 0) return fail("align_tile must be positive");
  if (tile % align_tile != 0) return fail("tile must be a multiple of align_tile");
  if (capacity < 0) return fail("capacity must be non-negative");
  if (num_tasks_i32 == nullptr) return fail("num_tasks pointer must be non-null");
  if (capacity > 0 && tasks_i32 == nullptr) return fail("tasks pointer must be non-null");
  if (groups > 0 && group_sizes == nullptr) return fail("group_sizes pointer must be non-null");
  if (!aligned(tasks_i32, 16)) return fail("tasks buffer must be 16-byte aligned");
  DeviceGuard guard(device_index);
  if (guard.error() != hipSuccess) return fail_hip("hipSetDevice", guard.error());
  const hipError_t err = shk::launch_group_info(group_sizes, groups, tile, align_tile, capacity, tasks_i32,
                                                num_tasks_i32, info_i64, reinterpret_cast<hipStream_t>(stream));
  if (err != hipSuccess) return fail_hip("group info launch", err);
  return 0;
}

int amd_strix_halo_kernels_ragged_workspace_bytes(int kernel_index, int32_t m, int32_t n, int32_t k_packed,
                                                  int32_t groups, uint64_t* bytes) {
  g_last_error.clear();
  if (bytes == nullptr) return fail("bytes must be non-null");
  const auto& t = table();
  if (kernel_index < 0 || kernel_index >= (int)t.size())
    return fail("kernel index " + std::to_string(kernel_index) + " is out of range");
  const shk_kernel_desc& d = t[kernel_index].d;
  if (d.family != SHK_FAMILY_RAGGED_FWD && d.family != SHK_FAMILY_RAGGED_BWD)
    return fail("kernel index " + std::to_string(kernel_index) + " is not a ragged kernel");
  if (m < 0 || n < 0 || k_packed < 0 || groups < 0) return fail("sizes must be non-negative");
  *bytes = ragged_workspace_bytes(d, m, n, k_packed, groups);
  return 0;
}

int amd_strix_halo_kernels_launch_ragged_fwd(int kernel_index, int device_index, uintptr_t stream,
                                             const void* lhs, const void* rhs, const void* a_scale,
                                             const void* b_scale, const int32_t* tasks_i32,
                                             const int32_t* num_tasks_i32, int32_t capacity, void* out, int32_t m,
                                             int32_t n, int32_t k_packed, int32_t groups, int32_t subchannel,
                                             int32_t out_mode) {
  return amd_strix_halo_kernels_launch_ragged_fwd_ws(kernel_index, device_index, stream, lhs, rhs, a_scale,
                                                     b_scale, tasks_i32, num_tasks_i32, capacity, out, m, n,
                                                     k_packed, groups, subchannel, out_mode, nullptr, 0);
}

namespace {

// The ragged forward; job: a task list for it to build first (in the fp6
// conversion launch where that holds the groups, else in its own launch),
// already validated.
int ragged_fwd(int kernel_index, int device_index, uintptr_t stream, const void* lhs, const void* rhs,
               const void* a_scale, const void* b_scale, const int32_t* tasks_i32, const int32_t* num_tasks_i32,
               int32_t capacity, void* out, int32_t m, int32_t n, int32_t k_packed, int32_t groups,
               int32_t subchannel, int32_t out_mode, void* workspace, uint64_t workspace_bytes,
               const shk::TaskJob* job) {
  g_last_error.clear();
  const Entry* e = nullptr;
  if (lookup(kernel_index, SHK_FAMILY_RAGGED_FWD, &e)) return 1;
  const shk_kernel_desc& d = e->d;
  const bool fp6 = d.operand_format == SHK_OPERANDS_FP6;
  if (lhs == nullptr || rhs == nullptr || a_scale == nullptr || b_scale == nullptr || out == nullptr ||
      tasks_i32 == nullptr || num_tasks_i32 == nullptr)
    return fail("lhs, rhs, scales, task list and out pointers must be non-null");
  if (m < 0 || n < 0 || k_packed < 0 || groups < 0 || capacity < 0) return fail("sizes must be non-negative");
  if (check_subchannel(d, subchannel)) return 1;
  if (check_out_mode(out_mode)) return 1;
  const int k = 2 * k_packed;
  if (!fp6 && d.scale_mode == SHK_SCALE_PER_CHANNEL && k > kMaxInt4AccK)
    return fail("int4 per-channel kernels support K <= " + std::to_string(kMaxInt4AccK));
  if (!aligned(tasks_i32, 16)) return fail("tasks buffer must be 16-byte aligned");
  if (fp6 && check_f6_ragged(d, subchannel, b_scale, out, m, n, k_packed, groups, workspace, workspace_bytes)) return 1;
  if (m == 0 || n == 0 || capacity == 0) {
    // nothing to multiply; a requested task list is still built
    if (job == nullptr) return 0;
    DeviceGuard guard(device_index);
    if (guard.error() != hipSuccess) return fail_hip("hipSetDevice", guard.error());
    const hipError_t err = shk::launch_group_info(job->sizes, job->groups, job->tile, job->align, job->capacity,
                                                  job->tasks, job->num_tasks, nullptr,
                                                  reinterpret_cast<hipStream_t>(stream));
    if (err != hipSuccess) return fail_hip("group info launch", err);
    return 0;
  }
  shk::RaggedFwdArgs p{};
  p.lhs = static_cast<const uint8_t*>(lhs);
  p.rhs = static_cast<const uint8_t*>(rhs);
  p.a_scale = static_cast<const uint16_t*>(a_scale);
  p.b_scale = static_cast<const uint16_t*>(b_scale);
  p.tasks = tasks_i32;
  p.num_tasks = num_tasks_i32;
  p.capacity = capacity;
  p.out = out;
  p.M = m;
  p.N = n;
  p.K = k;
  p.groups = groups;
  const bool a_km = d.layout == SHK_LAYOUT_NN || d.layout == SHK_LAYOUT_NT;
  const bool b_km = d.layout == SHK_LAYOUT_NT || d.layout == SHK_LAYOUT_TT;
  p.lda = a_km ? k_packed : m;
  p.ldb = b_km ? k_packed : n;
  p.subchannel = subchannel;
  p.scale_cols = subchannel > 0 ? (k + subchannel - 1) / subchannel : 1;
  p.out_mode = out_mode;
  p.a_aligned = a_km ? (aligned(lhs, 16) && p.lda % 16 == 0) : (aligned(lhs, 8) && p.lda % 8 == 0);
  p.b_aligned = b_km ? (aligned(rhs, 16) && p.ldb % 16 == 0) : (aligned(rhs, 8) && p.ldb % 8 == 0);
  p.out_vec = (n % 4 == 0) && aligned(out, 16) && aligned(b_scale, 8);
  p.layout = d.layout;
  p.work = static_cast<uint8_t*>(workspace);
  const long tiles_n = (n + d.block_n - 1) / d.block_n;
  const long grid = (long)capacity * tiles_n;
  if (grid > 0x7FFFFFFFL) return fail("ragged forward grid is too large");
  DeviceGuard guard(device_index);
  if (guard.error() != hipSuccess) return fail_hip("hipSetDevice", guard.error());
  const hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  if (job != nullptr) {
    if (fp6 && groups <= shk::kFusedTaskGroups) {
      p.job = *job;
    } else {
      const hipError_t err = shk::launch_group_info(job->sizes, job->groups, job->tile, job->align, job->capacity,
                                                    job->tasks, job->num_tasks, nullptr, s);
      if (err != hipSuccess) return fail_hip("group info launch", err);
    }
  }
  const hipError_t err = e->fwd(p, dim3((unsigned)grid), s);
  if (err != hipSuccess) return fail_hip("ragged forward launch", err);
  return 0;
}

}  // namespace

int amd_strix_halo_kernels_launch_ragged_fwd_ws(int kernel_index, int device_index, uintptr_t stream,
                                                const void* lhs, const void* rhs, const void* a_scale,
                                                const void* b_scale, const int32_t* tasks_i32,
                                                const int32_t* num_tasks_i32, int32_t capacity, void* out,
                                                int32_t m, int32_t n, int32_t k_packed, int32_t groups,
                                                int32_t subchannel, int32_t out_mode, void* workspace,
                                                uint64_t workspace_bytes) {
  return ragged_fwd(kernel_index, device_index, stream, lhs, rhs, a_scale, b_scale, tasks_i32, num_tasks_i32,
                    capacity, out, m, n, k_packed, groups, subchannel, out_mode, workspace, workspace_bytes, nullptr);
}

int amd_strix_halo_kernels_launch_ragged_fwd_grouped(int kernel_index, int device_index, uintptr_t stream,
                                                     const void* lhs, const void* rhs, const void* a_scale,
                                                     const void* b_scale, const int32_t* group_sizes,
                                                     int32_t align_tile, int32_t* tasks_i32, int32_t* num_tasks_i32,
                                                     int32_t capacity, void* out, int32_t m, int32_t n,
                                                     int32_t k_packed, int32_t groups, int32_t subchannel,
                                                     int32_t out_mode, void* workspace, uint64_t workspace_bytes) {
  g_last_error.clear();
  const Entry* e = nullptr;
  if (lookup(kernel_index, SHK_FAMILY_RAGGED_FWD, &e)) return 1;
  const int tile = e->d.block_m;
  if (groups < 0) return fail("groups must be non-negative");
  if (groups > shk::max_info_groups())
    return fail("at most " + std::to_string(shk::max_info_groups()) + " groups are supported");
  if (align_tile <= 0) return fail("align_tile must be positive");
  if (tile % align_tile != 0) return fail("the entry's task tile must be a multiple of align_tile");
  if (e->d.operand_format == SHK_OPERANDS_FP6 && align_tile % 32 != 0)
    return fail("fp6 ragged entries need align_tile a multiple of 32 (tasks start on a 32-row panel)");
  if (capacity < 0) return fail("capacity must be non-negative");
  // the device builds the list, so a list that could outgrow the buffer is
  // refused here: the forward would otherwise skip every task and leave out
  // unwritten
  const int32_t need = amd_strix_halo_kernels_ragged_task_capacity(m, groups, tile, align_tile);
  if (capacity < need)
    return fail("capacity " + std::to_string(capacity) + " is below the " + std::to_string(need) +
                " tasks the list may need for " + std::to_string(m) + " rows in " + std::to_string(groups) +
                " groups (amd_strix_halo_kernels_ragged_task_capacity)");
  if (num_tasks_i32 == nullptr || tasks_i32 == nullptr) return fail("task list pointers must be non-null");
  if (groups > 0 && group_sizes == nullptr) return fail("group_sizes pointer must be non-null");
  const shk::TaskJob job{group_sizes, groups, tile, align_tile, capacity, tasks_i32, num_tasks_i32, nullptr};
  return ragged_fwd(kernel_index, device_index, stream, lhs, rhs, a_scale, b_scale, tasks_i32, num_tasks_i32,
                    capacity, out, m, n, k_packed, groups, subchannel, out_mode, workspace, workspace_bytes, &job);
}

int amd_strix_halo_kernels_launch_ragged_bwd(int kernel_index, int device_index, uintptr_t stream,
                                             const void* lhs, const void* rhs, const void* a_scale,
                                             const void* b_scale, const int32_t* group_sizes, void* out,
                                             int32_t m, int32_t n, int32_t k_packed, int32_t groups,
                                             int32_t subchannel, int32_t split_k, int32_t out_mode) {
  return amd_strix_halo_kernels_launch_ragged_bwd_ws(kernel_index, device_index, stream, lhs, rhs, a_scale,
                                                     b_scale, group_sizes, out, m, n, k_packed, groups, subchannel,
                                                     split_k, out_mode, nullptr, 0);
}

int amd_strix_halo_kernels_launch_ragged_bwd_ws(int kernel_index, int device_index, uintptr_t stream,
                                                const void* lhs, const void* rhs, const void* a_scale,
                                                const void* b_scale, const int32_t* group_sizes, void* out,
                                                int32_t m, int32_t n, int32_t k_packed, int32_t groups,
                                                int32_t subchannel, int32_t split_k, int32_t out_mode,
                                                void* workspace, uint64_t workspace_bytes) {
  g_last_error.clear();
  const Entry* e = nullptr;
  if (lookup(kernel_index, SHK_FAMILY_RAGGED_BWD, &e)) return 1;
  const shk_kernel_desc& d = e->d;
  const bool fp6 = d.operand_format == SHK_OPERANDS_FP6;
  if (lhs == nullptr || rhs == nullptr || a_scale == nullptr || b_scale == nullptr || out == nullptr ||
      group_sizes == nullptr)
    return fail("lhs, rhs, scales, group_sizes and out pointers must be non-null");
  if (m < 0 || n < 0 || k_packed < 0 || groups < 0) return fail("sizes must be non-negative");
  if (split_k < 1 || split_k > 65535) return fail("split_k must be in [1, 65535]");
  if (check_subchannel(d, subchannel)) return 1;
  if (out_mode != SHK_OUT_F32 && out_mode != SHK_OUT_I32)
    return fail("ragged backward writes fp32 (or raw int32) output");
  const int k_cap = 2 * k_packed;
  if (!fp6 && d.scale_mode == SHK_SCALE_PER_CHANNEL && k_cap > kMaxInt4AccK)
    return fail("int4 per-channel kernels support K <= " + std::to_string(kMaxInt4AccK));
  if (fp6 && check_f6_ragged(d, subchannel, b_scale, out, m, n, k_packed, groups, workspace, workspace_bytes)) return 1;
  if (m == 0 || n == 0 || groups == 0) return 0;
  shk::RaggedBwdArgs p{};
  p.lhs = static_cast<const uint8_t*>(lhs);
  p.rhs = static_cast<const uint8_t*>(rhs);
  p.a_scale = static_cast<const uint16_t*>(a_scale);
  p.b_scale = static_cast<const uint16_t*>(b_scale);
  p.group_sizes = group_sizes;
  p.out = out;
  p.M = m;
  p.N = n;
  p.k_cap = k_cap;
  p.groups = groups;
  const bool a_km = d.layout == SHK_LAYOUT_NN || d.layout == SHK_LAYOUT_NT;
  const bool b_km = d.layout == SHK_LAYOUT_NT || d.layout == SHK_LAYOUT_TT;
  p.lda = a_km ? k_packed : m;
  p.ldb = b_km ? k_packed : n;
  p.subchannel = subchannel;
  p.scale_cols = subchannel > 0 ? (k_cap + subchannel - 1) / subchannel : 1;
  // fp6 entries compute each output whole: any split_k gives the result of
  // split_k = 1, which they write directly.
  p.split_k = fp6 ? 1 : split_k;
  p.out_mode = out_mode;
  p.a_aligned = a_km ? (aligned(lhs, 16) && p.lda % 16 == 0) : (aligned(lhs, 8) && p.lda % 8 == 0);
  p.b_aligned = b_km ? (aligned(rhs, 16) && p.ldb % 16 == 0) : (aligned(rhs, 8) && p.ldb % 8 == 0);
  p.out_vec = (n % 4 == 0) && aligned(out, 16) && aligned(b_scale, 8);
  p.layout = d.layout;
  p.work = static_cast<uint8_t*>(workspace);
  const long tiles = (long)groups * ((m + d.block_m - 1) / d.block_m) * ((n + d.block_n - 1) / d.block_n);
  if (tiles > 0x7FFFFFFFL) return fail("ragged backward grid is too large");
  DeviceGuard guard(device_index);
  if (guard.error() != hipSuccess) return fail_hip("hipSetDevice", guard.error());
  const hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  hipError_t err = e->bwd(p, dim3((unsigned)tiles, (unsigned)p.split_k), s);
  if (err != hipSuccess) return fail_hip("ragged backward launch", err);
  if (p.split_k > 1 && d.scale_mode == SHK_SCALE_PER_CHANNEL && out_mode == SHK_OUT_F32) {
    err = shk::launch_bwd_finalize(static_cast<float*>(out), p.a_scale, p.b_scale, groups, m, n, s);
    if (err != hipSuccess) return fail_hip("ragged backward finalize launch", err);
  }
  return 0;
}

int amd_strix_halo_kernels_quantize(int device_index, uintptr_t stream, const void* x, int32_t src, int64_t rows,
                                    int64_t cols, int64_t ld_x, float inv_scale, int32_t bits, int32_t mode,
                                    void* out, int64_t ld_out) {
  g_last_error.clear();
  if (src < SHK_SRC_F32 || src > SHK_SRC_I8) return fail("unknown source type " + std::to_string(src));
  if (mode < SHK_QUANT_CODES || mode > SHK_QUANT_PACK_ROWS) return fail("unknown quantize mode " + std::to_string(mode));
  if (bits != 4 && bits != 8) return fail("bits must be 4 or 8");
  if (mode != SHK_QUANT_CODES && bits != 4) return fail("only int4 codes are packed (bits must be 4)");
  if (src == SHK_SRC_I8 && mode == SHK_QUANT_CODES) return fail("int8 sources are codes already; pack them");
  if (src != SHK_SRC_I8 && !(inv_scale > 0.0f)) return fail("inv_scale must be positive");
  if (rows < 0 || cols < 0) return fail("rows and cols must be non-negative");
  const int64_t out_rows = mode == SHK_QUANT_PACK_ROWS ? (rows + 1) / 2 : rows;
  const int64_t out_cols = mode == SHK_QUANT_PACK_COLS ? (cols + 1) / 2 : cols;
  if (ld_x < cols) return fail("ld_x must be at least cols");
  if (ld_out < out_cols) return fail("ld_out must be at least the output row length");
  if (rows == 0 || cols == 0) return 0;
  if (x == nullptr || out == nullptr) return fail("x and out pointers must be non-null");
  DeviceGuard guard(device_index);
  if (guard.error() != hipSuccess) return fail_hip("hipSetDevice", guard.error());
  const shk::QuantArgs p{x,        static_cast<uint8_t*>(out), rows, cols, ld_x, ld_out, out_rows, out_cols,
                         inv_scale, bits,                       src,  mode};
  const hipError_t err = shk::launch_quantize(p, reinterpret_cast<hipStream_t>(stream));
  if (err == hipErrorInvalidValue) return fail("quantize grid is too large");
  if (err != hipSuccess) return fail_hip("quantize launch", err);
  return 0;
}

}  // extern "C"
