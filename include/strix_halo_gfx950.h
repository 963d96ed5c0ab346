/*
 * C ABI of the gfx950 (MI355X) quantized GEMM library
 * (libamd_strix_halo_kernels_gfx950.so).
 *
 * This library replaces the reference's HSACO loader/dispatcher
 * (native/src/dispatch.cpp) and its per-kernel JSON launch metadata
 * (the kernels/amdgcn JSON files) with kernels compiled into the library and a static
 * kernel table.  The Python host layer (amd_strix_halo_kernels.native) binds
 * these symbols with ctypes.
 *
 * Conventions (same as the reference dispatcher, dispatch.cpp:18-23,220-222):
 *   - every launch function returns 0 on success and 1 on failure;
 *   - on failure amd_strix_halo_kernels_last_error() returns a message that
 *     stays valid until the next call on the same thread;
 *   - all device pointers are borrowed; the library never allocates or frees
 *     device memory; workspaces are passed in by the caller (except for
 *     amd_strix_halo_kernels_launch_gemm_noalloc, whose workspace is a static
 *     array of the library's code object);
 *   - launches are asynchronous on the given stream (a hipStream_t passed as
 *     uintptr_t, 0 = the null stream) on device `device_index`; the calling
 *     thread's current device is restored before returning.
 * Kernels are selected by table index (amd_strix_halo_kernels_kernel_table_*);
 * the library derives grid, block and LDS size from the table entry.
 */
#ifndef STRIX_HALO_GFX950_H
#define STRIX_HALO_GFX950_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Kernel families in the table. */
#define SHK_FAMILY_DENSE 0
#define SHK_FAMILY_RAGGED_FWD 1
#define SHK_FAMILY_RAGGED_BWD 2

/* Layouts (reference metadata.GemmLayout, metadata.py:35-45). */
#define SHK_LAYOUT_NN 0
#define SHK_LAYOUT_NT 1
#define SHK_LAYOUT_TN 2
#define SHK_LAYOUT_TT 3

/* Scale modes (reference metadata.ScaleMode, metadata.py:24-26). */
#define SHK_SCALE_PER_CHANNEL 0
#define SHK_SCALE_SUBCHANNEL 1

/* Epilogue kinds of a table entry: PLAIN serves Epilogue.NONE and
 * Epilogue.RELU2 (chosen per launch), SWIGLU serves Epilogue.SWIGLU. */
#define SHK_EPI_KIND_PLAIN 0
#define SHK_EPI_KIND_SWIGLU 2

/* Per-launch epilogue (reference metadata.Epilogue, metadata.py:29-32). */
#define SHK_EPILOGUE_NONE 0
#define SHK_EPILOGUE_RELU2 1
#define SHK_EPILOGUE_SWIGLU 2

/* Output modes.  BF16 and F32 hold the scaled result; I32 writes the exact
 * int32 accumulators (the integer matmul before any scale) for verification:
 * for SwiGLU entries the I32 output is [M, 2*D] with up columns then gate
 * columns; for subchannel entries it is the int32 sum over all K. */
#define SHK_OUT_BF16 0
#define SHK_OUT_F32 1
#define SHK_OUT_I32 2

/* Operand formats of a dense entry.  PACKED kernels read A and B as given;
 * FP6 kernels (int4 only) first convert both operands into a caller
 * workspace of amd_strix_halo_kernels_gemm_workspace_bytes() bytes: every
 * int4 value v is exact as v/8 in the 6-bit float e2m3, whose MFMA runs at
 * twice the int8 rate; one fp32 pass is exact for K <= 262144, and
 * per-channel calls with a longer K (up to 2^24) run in exact K slices of
 * 262144 whose int32 sums add in the workspace before one pass applies the
 * scales and the epilogue.  The int8 engines' int4 per-channel entries hold
 * x16-widened products and need K < 131072 per int32 accumulator (per K
 * slice for split-K entries). */
#define SHK_OPERANDS_PACKED 0
#define SHK_OPERANDS_FP6 1
/* STREAM entries (block_m 16, 32, 64; block_k 32) read the packed operands
 * straight from HBM like PACKED ones.  Per-channel calls may split a tile's
 * K over several workgroups that add exact int32 partials; they do so only
 * with a workspace of amd_strix_halo_kernels_gemm_workspace_bytes() bytes
 * (0 when the shape needs no split), which must be zero before the first
 * launch that uses it; every completed launch leaves all of it that it used
 * zero (arrival counters and partials alike), so a zero-filled workspace can
 * be reused by launches of any shape in stream order (not by launches that
 * overlap in time).  Without a
 * workspace (amd_strix_halo_kernels_launch_gemm) the tile's K stays in one
 * workgroup, which limits int4 per-channel calls to K <= 523776.  Results
 * are identical either way. */
#define SHK_OPERANDS_STREAM 2

/* Tile schedules of a dense entry (reference metadata.KernelSchedule,
 * metadata.py:51-53).  STANDARD launches one workgroup per output tile;
 * PERSISTENT launches one workgroup per resident slot (occupancy x CUs,
 * a multiple of 8 so each workgroup keeps its XCD, at most the tile count),
 * each taking every gridDim-th tile in the same XCD-aware order. */
#define SHK_SCHEDULE_STANDARD 0
#define SHK_SCHEDULE_PERSISTENT 1

/* Sources of amd_strix_halo_kernels_quantize: float values to quantize, or
 * existing int8 codes to pack. */
#define SHK_SRC_F32 0
#define SHK_SRC_F16 1
#define SHK_SRC_BF16 2
#define SHK_SRC_I8 3

/* Outputs of amd_strix_halo_kernels_quantize. */
#define SHK_QUANT_CODES 0     /* int8 codes, rows x cols */
#define SHK_QUANT_PACK_COLS 1 /* int4 pairs along each row: rows x ceil(cols/2) bytes */
#define SHK_QUANT_PACK_ROWS 2 /* int4 pairs of rows 2r, 2r+1: ceil(rows/2) x cols bytes */

typedef struct shk_kernel_desc {
  int32_t index;
  int32_t family;          /* SHK_FAMILY_* */
  int32_t dtype_bits;      /* 4 (packed int4) or 8 (int8) */
  int32_t layout;          /* SHK_LAYOUT_* */
  int32_t scale_mode;      /* SHK_SCALE_* */
  int32_t min_subchannel;  /* smallest subchannel size served (subchannel entries) */
  int32_t max_subchannel;  /* largest subchannel size served (subchannel entries) */
  int32_t epilogue_kind;   /* SHK_EPI_KIND_* */
  int32_t block_m;         /* output rows per workgroup (ragged fwd: task rows) */
  int32_t block_n;         /* output columns per workgroup */
  int32_t block_k;         /* logical K per LDS stage */
  int32_t num_waves;       /* 64-lane waves per workgroup */
  int32_t num_stages;      /* LDS stages (double buffered = 2) */
  int32_t lds_bytes;       /* LDS per workgroup */
  int32_t group_size_m;    /* tile-row swizzle width (dense) */
  int32_t operand_format;  /* SHK_OPERANDS_* */
  int32_t schedule;        /* SHK_SCHEDULE_* */
  int32_t split_k;         /* K slices per output tile (dense); > 1: float32 output.  PACKED
                              entries add the slices into it with hardware float atomics, so
                              `out` must hold zeros and be coarse-grained device memory
                              (hipMalloc, torch's allocator); the slices add in a run-dependent
                              order, so the last bits of a result may differ from run to run.
                              STREAM entries compute each output whole (exact int32 sums) and
                              store it: split_k sets only the K multiple and the output type */
} shk_kernel_desc;

/* ---- status (reference dispatch.cpp:206-222) ---------------------------- */

/* Replaces amd_strix_halo_kernels_dispatch_version (dispatch.cpp:206).
 * Version 2 = gfx950 table-driven dispatch. */
int amd_strix_halo_kernels_dispatch_version(void);

/* Replaces amd_strix_halo_kernels_has_compiled_code_objects
 * (dispatch.cpp:208-210): 1, the gfx950 code objects are linked in. */
int amd_strix_halo_kernels_has_compiled_code_objects(void);

/* Replaces amd_strix_halo_kernels_has_hip_runtime (dispatch.cpp:212-214):
 * 1 when the HIP runtime reports at least one device. */
int amd_strix_halo_kernels_has_hip_runtime(void);

/* Replaces amd_strix_halo_kernels_has_linked_kernels (dispatch.cpp:216-218):
 * 1 when a gfx950 device is present to run the linked kernels. */
int amd_strix_halo_kernels_has_linked_kernels(void);

/* Replaces amd_strix_halo_kernels_last_error (dispatch.cpp:220-222). */
const char* amd_strix_halo_kernels_last_error(void);

/* Target architecture string of the linked code objects ("gfx950"). */
const char* amd_strix_halo_kernels_arch(void);

/* ---- kernel table (replaces the kernels/amdgcn JSON metadata and the registry tile
 * seeds, registry.py:112-176, read by native.py:165-169) ----------------- */

int amd_strix_halo_kernels_kernel_table_size(void);
/* Copies entry `index` into *out.  Returns 0, or 1 for a bad index. */
int amd_strix_halo_kernels_kernel_table_entry(int index, shk_kernel_desc* out);

/* The dense entry the Python registry's select() picks (registry.py:254-352
 * of the reference: same dtype, scale, epilogue, layout, schedule and
 * split-K; the shape a tile multiple within the entry's K bound; the
 * largest (measured throughput, block_m * block_n), the first on ties), for
 * a caller that keeps the reference's own registry: the fields of its
 * KernelMetadata, whose gfx1151 tiles have no entry here, and the call's
 * logical shape map to a gfx950 table index.  dtype_bits 4 or 8; layout
 * SHK_LAYOUT_*; subchannel 0 (per-channel) or 32..256; epilogue
 * SHK_EPILOGUE_*; schedule SHK_SCHEDULE_*; split_k 0 for any, else the
 * kernel's split.  Writes *kernel_index and returns 0, or returns 1 with
 * last_error ("no kernel for ...") when no entry fits.  No counterpart in
 * the reference, whose bridge (native.py:690-767) is handed a gfx1151
 * table entry directly. */
int amd_strix_halo_kernels_select_dense(int32_t dtype_bits, int32_t layout, int32_t subchannel, int32_t epilogue,
                                        int32_t schedule, int32_t split_k, int32_t m, int32_t n, int32_t k,
                                        int32_t* kernel_index);

/* ---- dense GEMM -----------------------------------------------------------
 * Replaces amd_strix_halo_kernels_launch_hsaco (dispatch.cpp:224-283) as
 * called by native.launch_generated_kernel (native.py:690-767).
 * Computes out = epilogue(scale(A @ B)) for logical shape (m, n, k), with
 * A/B packed int4 (two nibbles per byte along K) or int8 per the entry's
 * dtype and layout (NN: A[m, k'], B[k', b_cols]; NT: B[b_cols, k'];
 * TN: A[k', m]; k' = k/2 for int4).  b_cols = n, or 2*n for SwiGLU entries
 * where B holds [up | gate].  Scales are bf16: per-channel a_scale[m],
 * b_scale[b_cols]; subchannel S: a_scale[m, ceil(k/S)],
 * b_scale[ceil(k/S), b_cols].  Requires m % block_m == 0, n % block_n == 0,
 * k % block_k == 0 and (subchannel) k % S == 0 (reference
 * template_config.py:22-38).  `gate` of the reference signature is dropped:
 * SwiGLU is fused.  Entries with operand_format SHK_OPERANDS_FP6 need a
 * workspace and are launched with amd_strix_halo_kernels_launch_gemm_ws;
 * this function refuses them. */
int amd_strix_halo_kernels_launch_gemm(int kernel_index, int device_index, uintptr_t stream,
                                       const void* a, const void* b, const void* a_scale,
                                       const void* b_scale, void* out, int32_t m, int32_t n,
                                       int32_t k, int32_t subchannel, int32_t epilogue,
                                       int32_t out_mode);

/* Workspace bytes a dense entry needs for shape (m, n, k) (0 for PACKED
 * entries), written to *bytes.  Returns 0, or 1 for a bad index or shape.
 * No counterpart in the reference, whose gfx1151 kernels read int4 operands
 * directly. */
int amd_strix_halo_kernels_gemm_workspace_bytes(int kernel_index, int32_t m, int32_t n, int32_t k,
                                                uint64_t* bytes);

/* amd_strix_halo_kernels_launch_gemm with a caller workspace (16-byte
 * aligned, at least amd_strix_halo_kernels_gemm_workspace_bytes() bytes; may
 * be null for PACKED entries).  The workspace is overwritten by the launch
 * and may be reused once the launch has completed in stream order.  Same
 * reference interface as amd_strix_halo_kernels_launch_gemm. */
int amd_strix_halo_kernels_launch_gemm_ws(int kernel_index, int device_index, uintptr_t stream,
                                          const void* a, const void* b, const void* a_scale,
                                          const void* b_scale, void* out, int32_t m, int32_t n,
                                          int32_t k, int32_t subchannel, int32_t epilogue,
                                          int32_t out_mode, void* workspace, uint64_t workspace_bytes);

/* Size of the library's scratch array (per device): the largest fp6 operand
 * workspace amd_strix_halo_kernels_launch_gemm_noalloc accepts, 128 MiB
 * (0.75 byte per value of A and B: covers M*K + b_cols*K <= 178956970
 * values, e.g. M = N = K = 8192). */
#define SHK_NOALLOC_SCRATCH_BYTES (128u * 1024u * 1024u)

/* amd_strix_halo_kernels_launch_gemm_ws without a workspace argument, for
 * callers that cannot allocate device memory (code under HIP graph capture,
 * tight serving loops, harnesses that forbid hipMalloc).  No counterpart in
 * the reference.  FP6 entries convert their operands into the library's own
 * static scratch array of SHK_NOALLOC_SCRATCH_BYTES on `device_index`
 * instead of a caller workspace; STREAM entries that split K keep their
 * arrival counters and partials there and clear the counters with a small
 * kernel on `stream` before the GEMM (two launches); PACKED entries need
 * none and run as amd_strix_halo_kernels_launch_gemm.  The array is reserved
 * on every device where the library's code object is loaded, whether or not
 * this entry point is called.  The call allocates and frees nothing (its
 * first call on a device looks the array's address up once).  Shapes whose
 * workspace (amd_strix_halo_kernels_gemm_workspace_bytes) exceeds
 * SHK_NOALLOC_SCRATCH_BYTES are rejected with rc 1.  Every call on a device
 * shares that device's array: the conversion (or the counter clear and the
 * partial stores) rewrites every byte the GEMM reads before it reads it, so
 * no state carries over from an earlier call, but calls that overlap in time
 * on one device (different streams, or threads without stream ordering) race
 * on the array and give undefined results.  Same arguments, validation and
 * errors as amd_strix_halo_kernels_launch_gemm. */
int amd_strix_halo_kernels_launch_gemm_noalloc(int kernel_index, int device_index, uintptr_t stream,
                                               const void* a, const void* b, const void* a_scale,
                                               const void* b_scale, void* out, int32_t m, int32_t n,
                                               int32_t k, int32_t subchannel, int32_t epilogue,
                                               int32_t out_mode);

/* The two halves of a fp6 launch, for callers that convert an operand once
 * and multiply it many times (a weight matrix), and for timing the GEMM
 * kernel on its own.  amd_strix_halo_kernels_gemm_convert converts operand 0
 * (A, laid out as for launch_gemm) or operand 1 (B) of shape (m, n, k) into
 * its part of the workspace; amd_strix_halo_kernels_launch_gemm_converted
 * runs the GEMM on the converted operands in the workspace.  A launch_gemm_ws
 * call is exactly convert(A), convert(B), launch_gemm_converted on one stream.
 * Both refuse PACKED entries.  No counterpart in the reference. */
int amd_strix_halo_kernels_gemm_convert(int kernel_index, int device_index, uintptr_t stream, int32_t operand,
                                        const void* src, int32_t m, int32_t n, int32_t k, void* workspace,
                                        uint64_t workspace_bytes);
int amd_strix_halo_kernels_launch_gemm_converted(int kernel_index, int device_index, uintptr_t stream,
                                                 const void* a_scale, const void* b_scale, void* out, int32_t m,
                                                 int32_t n, int32_t k, int32_t epilogue, int32_t out_mode,
                                                 const void* workspace, uint64_t workspace_bytes);

/* ---- ragged task list -------------------------------------------------------
 * Device-side replacement of calculate_group_info (ragged.py:201-323, the
 * Triton kernel ragged.py:127-185).  From int32 group_sizes[groups] builds,
 * for tasks t < capacity:
 *   tasks_i32[4*t + {0,1,2,3}] = group_id, block_start, actual_start, actual_end
 * and writes num_tasks to *num_tasks_i32; slots t >= num_tasks are zero.
 * If info_i64 is non-null it also receives the six int64 arrays of
 * RaggedGroupInfo, each `capacity` long, in the order group_id, block_start,
 * actual_start, actual_end, start_within_block, actual_size.
 * Negative sizes count as zero (torch.clamp(min=0), ragged.py:256).
 * If the tasks do not fit in `capacity`, *num_tasks_i32 receives the true
 * count, the arrays receive the first `capacity` tasks, and the ragged
 * forward refuses to run any task (the caller sizes capacity with
 * amd_strix_halo_kernels_ragged_task_capacity). */
int amd_strix_halo_kernels_ragged_group_info(int device_index, uintptr_t stream,
                                             const int32_t* group_sizes, int32_t groups,
                                             int32_t tile, int32_t align_tile, int32_t capacity,
                                             int32_t* tasks_i32, int32_t* num_tasks_i32,
                                             int64_t* info_i64);

/* Upper bound on the number of row tasks for `rows` rows in `groups` groups. */
int32_t amd_strix_halo_kernels_ragged_task_capacity(int32_t rows, int32_t groups, int32_t tile,
                                                    int32_t align_tile);

/* ---- ragged forward ---------------------------------------------------------
 * Replaces amd_strix_halo_kernels_launch_ragged_fwd_hsaco (dispatch.cpp:286-389)
 * as called by native.launch_ragged_fwd_kernel (native.py:533-600).
 * out[rows of group g, :] = lhs[rows, :] @ rhs[g] with the task list built
 * above (tasks_i32 / num_tasks_i32 device pointers, `capacity` slots; the
 * grid covers capacity tasks and tasks >= *num_tasks_i32 exit).
 * Layouts: NN lhs[m, k'], rhs[G, k', n]; NT rhs[G, n, k']; TN lhs[k', m];
 * TT both.  Scales bf16: per-channel a_scale[m], b_scale[G, n]; subchannel S
 * a_scale[m, ceil(k/S)], b_scale[G, ceil(k/S), n].  out_mode BF16 or F32
 * (or I32 raw) [m, n].  The entry's block_m must equal the task tile.
 * FP6 entries (operand_format) need a workspace: they fail here and run
 * through amd_strix_halo_kernels_launch_ragged_fwd_ws. */
int amd_strix_halo_kernels_launch_ragged_fwd(int kernel_index, int device_index, uintptr_t stream,
                                             const void* lhs, const void* rhs, const void* a_scale,
                                             const void* b_scale, const int32_t* tasks_i32,
                                             const int32_t* num_tasks_i32, int32_t capacity,
                                             void* out, int32_t m, int32_t n, int32_t k_packed,
                                             int32_t groups, int32_t subchannel, int32_t out_mode);

/* ---- fp6 ragged entries -----------------------------------------------------
 * No counterpart in the reference (its ragged kernels read the packed
 * operands directly).  FP6 ragged entries convert both int4 operands into
 * the fp6 block format in a caller workspace of
 * amd_strix_halo_kernels_ragged_workspace_bytes bytes (0 for PACKED
 * entries; sizes as passed to the launch), 16-byte aligned, then run the
 * 128 x 128 fp6 GEMM.  Each family has a per-channel and a subchannel
 * (groups of 32 to 256) entry per layout.  They take N a multiple of 8,
 * K <= 262144, out 16-byte and b_scale 8-byte aligned (lhs and rhs in any
 * alignment); subchannel: M * ceil(K/S) even, and ceil(K/32) even for
 * groups of 32; the subchannel entries' workspace pads K to 256.
 * Forward: task list built with tile 128 (the entry's block_m) and an
 * align_tile that is a multiple of 32.  Backward: split_k has no effect
 * (each output is computed whole and written, the result of split_k = 1).
 * Otherwise the _ws calls equal the calls above, which they replace for
 * every entry. */
int amd_strix_halo_kernels_ragged_workspace_bytes(int kernel_index, int32_t m, int32_t n, int32_t k_packed,
                                                  int32_t groups, uint64_t* bytes);
int amd_strix_halo_kernels_launch_ragged_fwd_ws(int kernel_index, int device_index, uintptr_t stream,
                                                const void* lhs, const void* rhs, const void* a_scale,
                                                const void* b_scale, const int32_t* tasks_i32,
                                                const int32_t* num_tasks_i32, int32_t capacity,
                                                void* out, int32_t m, int32_t n, int32_t k_packed,
                                                int32_t groups, int32_t subchannel, int32_t out_mode,
                                                void* workspace, uint64_t workspace_bytes);

/* The task list and the forward in one call: the same as
 * amd_strix_halo_kernels_ragged_group_info(group_sizes, groups, tile = the
 * entry's block_m, align_tile, capacity, tasks_i32, num_tasks_i32, NULL)
 * followed by amd_strix_halo_kernels_launch_ragged_fwd_ws with that list.
 * No counterpart in the reference, whose forward takes the list from
 * calculate_group_info (ragged.py:201-323) as a separate step: the fp6
 * entries build it inside their conversion launch (up to 1024 groups), so
 * a call is two launches with no host work between them.  capacity must be
 * at least amd_strix_halo_kernels_ragged_task_capacity(m, groups, block_m,
 * align_tile) (rc 1 otherwise), the bound of any list those group sizes
 * can make, since the sizes are read on the device. */
int amd_strix_halo_kernels_launch_ragged_fwd_grouped(int kernel_index, int device_index, uintptr_t stream,
                                                     const void* lhs, const void* rhs, const void* a_scale,
                                                     const void* b_scale, const int32_t* group_sizes,
                                                     int32_t align_tile, int32_t* tasks_i32, int32_t* num_tasks_i32,
                                                     int32_t capacity, void* out, int32_t m, int32_t n,
                                                     int32_t k_packed, int32_t groups, int32_t subchannel,
                                                     int32_t out_mode, void* workspace, uint64_t workspace_bytes);

/* ---- ragged backward --------------------------------------------------------
 * Replaces amd_strix_halo_kernels_launch_ragged_bwd_hsaco (dispatch.cpp:391-457)
 * as called by native.launch_ragged_bwd_kernel (native.py:603-667).
 * out[g] = op(lhs[g]) @ op(rhs[g]) over the first group_sizes[g] (int32,
 * device) logical K values; K beyond group_sizes[g] reads as zero, including
 * the high nibble of an odd length (ragged.py:734-739).  Layouts: NN
 * lhs[G, m, k'], rhs[G, k', n]; NT rhs[G, n, k']; TN lhs[G, k', m].
 * Scales bf16: per-channel a_scale[G, m], b_scale[G, n]; subchannel S
 * a_scale[G, m, ceil(2k'/S)], b_scale[G, ceil(2k'/S), n].  out is fp32
 * [G, m, n].  split_k > 1 requires `out` to be zero-filled by the caller
 * (as the reference does, ragged.py:1330-1331): per-channel splits add exact
 * int32 partials and a finalize pass applies the scales (result identical to
 * split_k = 1); subchannel splits own whole scale groups and add fp32
 * partials atomically. */
int amd_strix_halo_kernels_launch_ragged_bwd(int kernel_index, int device_index, uintptr_t stream,
                                             const void* lhs, const void* rhs, const void* a_scale,
                                             const void* b_scale, const int32_t* group_sizes,
                                             void* out, int32_t m, int32_t n, int32_t k_packed,
                                             int32_t groups, int32_t subchannel, int32_t split_k,
                                             int32_t out_mode);
/* The backward with a workspace (fp6 ragged entries above). */
int amd_strix_halo_kernels_launch_ragged_bwd_ws(int kernel_index, int device_index, uintptr_t stream,
                                                const void* lhs, const void* rhs, const void* a_scale,
                                                const void* b_scale, const int32_t* group_sizes,
                                                void* out, int32_t m, int32_t n, int32_t k_packed,
                                                int32_t groups, int32_t subchannel, int32_t split_k,
                                                int32_t out_mode, void* workspace, uint64_t workspace_bytes);

/* Fake quantization and int4 packing on the device, in one pass over HBM.
 * No counterpart in the reference's dispatcher: its quant.py:14-51
 * (fake_quant_int, pack_int4_k_major) does this with torch element-wise ops,
 * which this replaces for device tensors.
 * x holds rows x cols values (row pitch ld_x elements) of type `src`.
 * For a float source the code of value v is
 *   clamp(rint(v * inv_scale), -2^(bits-1), 2^(bits-1) - 1)
 * with rint rounding half to even and NaN giving 0, which is what torch's
 * clamp(round(x.float() / scale)).to(int8) computes on the GPU: it divides
 * by a Python scalar by multiplying with its reciprocal, rounded once to
 * fp32 from double, so the caller passes inv_scale = (float)(1.0 / scale).
 * For SHK_SRC_I8 the codes are the source bytes, packed as given (their low
 * nibbles), as pack_int4_k_major does; bits must be 4 and mode a PACK mode.
 * PACK modes put the even element in the low nibble and the odd one in the
 * high nibble; an odd count pads with a zero element.  out has row pitch
 * ld_out bytes; bits is 4 for the PACK modes and 4 or 8 for CODES. */
int amd_strix_halo_kernels_quantize(int device_index, uintptr_t stream, const void* x, int32_t src, int64_t rows,
                                    int64_t cols, int64_t ld_x, float inv_scale, int32_t bits, int32_t mode,
                                    void* out, int64_t ld_out);

#ifdef __cplusplus
}
#endif

#endif /* STRIX_HALO_GFX950_H */
