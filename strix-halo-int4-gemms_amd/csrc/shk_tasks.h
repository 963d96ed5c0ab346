// Ragged task list on the device (calculate_group_info, ragged.py:201-323;
// the Triton kernel ragged.py:127-185).  One workgroup of NT threads: a
// blocked exclusive scan over the groups gives each group's first row and
// first task (kept in LDS), then every task slot binary-searches its group.
// Used by the stand-alone task-list launch (1024 threads, up to 16384
// groups) and by the fp6 conversion launch, whose first workgroup (256
// threads) builds the list beside the conversion for up to
// kFusedTaskGroups groups.
#pragma once

#include "shk_common.h"

namespace shk {

// Largest group count whose task list the fp6 conversion launch builds (its
// 16 KiB of LDS hold both per-group arrays).
constexpr int kFusedTaskGroups = 1024;

// What a task-list build writes: tasks[4 t + {0,1,2,3}] = group, block_start,
// actual_start, actual_end for t < capacity (zero past the count), the count
// in *num_tasks and, when info is non-null, the six int64 arrays of
// RaggedGroupInfo (each `capacity` long).  sizes == nullptr: no build.
struct TaskJob {
  const int32_t* sizes;
  int groups, tile, align, capacity;
  int32_t* tasks;
  int32_t* num_tasks;
  int64_t* info;
};

// Exclusive scan of one value per thread over the NT threads of the
// workgroup; *total receives the sum.  scratch: NT / 64 ints of LDS.
template <int NT>
__device__ __forceinline__ int block_exclusive_scan(int v, int* scratch, int& total) {
  static_assert(NT % 64 == 0 && NT <= 64 * 64, "whole waves, one scan wave");
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  int x = v;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const int y = __shfl_up(x, off, 64);
    if (lane >= off) x += y;
  }
  if (lane == 63) scratch[wave] = x;
  __syncthreads();
  if (wave == 0) {
    int w = lane < NT / 64 ? scratch[lane] : 0;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
      const int y = __shfl_up(w, off, 64);
      if (lane >= off) w += y;
    }
    if (lane < NT / 64) scratch[lane] = w;
  }
  __syncthreads();
  const int prefix = wave > 0 ? scratch[wave - 1] : 0;
  total = scratch[NT / 64 - 1];
  __syncthreads();
  return prefix + x - v;
}

// starts / task_starts: groups + 1 ints of LDS each; scratch: NT / 64 ints.
// Negative sizes count as zero (torch.clamp(min=0), ragged.py:256).
template <int NT>
__device__ void build_task_list(const TaskJob& j, int* starts, int* task_starts, int* scratch) {
  const int tid = threadIdx.x;
  const int groups = j.groups, tile = j.tile, align = j.align;
  int row_carry = 0, task_carry = 0;
  for (int base = 0; base < groups; base += NT) {
    const int g = base + tid;
    int sz = g < groups ? j.sizes[g] : 0;
    sz = sz < 0 ? 0 : sz;
    int row_total;
    const int row_ex = block_exclusive_scan<NT>(sz, scratch, row_total);
    const int start = row_carry + row_ex;
    const int aligned = (start / align) * align;
    const int blocks = sz == 0 ? 0 : (start + sz - aligned + tile - 1) / tile;
    int task_total;
    const int task_ex = block_exclusive_scan<NT>(blocks, scratch, task_total);
    if (g < groups) {
      starts[g] = start;
      task_starts[g] = task_carry + task_ex;
    }
    row_carry += row_total;
    task_carry += task_total;
  }
  if (tid == 0) {
    starts[groups] = row_carry;
    task_starts[groups] = task_carry;
    *j.num_tasks = task_carry;
  }
  __syncthreads();
  const int ntasks = task_carry;
  for (int t = tid; t < j.capacity; t += NT) {
    int gid = 0, bstart = 0, astart = 0, aend = 0;
    if (t < ntasks) {
      // the last group g with task_starts[g] <= t: upper bound over
      // task_starts[1..groups] (empty groups own no task)
      int lo = 0, hi = groups;
      while (lo < hi) {
        const int mid = (lo + hi) >> 1;
        if (task_starts[mid + 1] <= t) lo = mid + 1;
        else hi = mid;
      }
      gid = lo < groups ? lo : groups - 1;
      const int gstart = starts[gid];
      const int gend = starts[gid + 1];
      const int aligned = (gstart / align) * align;
      bstart = aligned + (t - task_starts[gid]) * tile;
      astart = bstart > gstart ? bstart : gstart;
      aend = (bstart + tile) < gend ? (bstart + tile) : gend;
    }
    *reinterpret_cast<int4*>(j.tasks + 4 * t) = make_int4(gid, bstart, astart, aend);
    if (j.info != nullptr) {
      const int size = aend > astart ? aend - astart : 0;
      const long cap = j.capacity;
      j.info[t] = gid;
      j.info[cap + t] = bstart;
      j.info[2 * cap + t] = astart;
      j.info[3 * cap + t] = aend;
      j.info[4 * cap + t] = astart - bstart;
      j.info[5 * cap + t] = size;
    }
  }
}

}  // namespace shk
