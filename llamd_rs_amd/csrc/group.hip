// group.hip -- expert grouping for the prefill path.
//
// The design of the reference's moe_group.comp (crates/llamd-vulkan/shaders/
// moe_group.comp:37-82) on one gfx950 workgroup: a counting sort of the
// n_tok * n_used (token, slot) pairs by expert -- LDS histogram, prefix sum,
// scatter -- giving each expert a contiguous run of pairs. The order of pairs
// inside one expert's run depends on atomic arrival, which is harmless: each
// pair's result is computed independently and written to its own output row
// (the pair index), so the expert-major result equals the token-major one
// exactly, the property crates/llamd-testing/tests/vulkan_prefill.rs:268-333
// holds the reference's Vulkan path to.
//
// Outputs (all experts are groups, empty ones included):
//   grp_expert[e] = e, grp_start[e], grp_count[e],
//   sub_start[0..n_expert] = prefix sum of ceil(count/16) (16-token chunks
//   of the batched kernel), followed by twin_start = sub_start[n_expert + 1
//   .. 2 n_expert + 1] = prefix sum of ceil(chunks/2) (twins: two chunks of
//   one expert, the work items of the twin batched kernel), slot_of_pair[p] = the chunk slot of pair p
//   (chunk sub_start[e] + j / 16, token j % 16 for the j-th pair of expert
//   e), pair_idx[i] = the pair index t * n_used + k at sorted position i.
// With max_chunks > 0, sub_start continues with a record per chunk,
// sub_info[max_chunks], then one per twin, twin_info[max_chunks] (GroupItem,
// launch.hpp): a wave of the batched kernels reads its work item in one load
// instead of a binary search of dependent loads and the group's fields.
#include "common.hpp"
#include "launch.hpp"

namespace llamd {
namespace {

constexpr int GROUP_MAX_EXPERTS = 1024;

__global__ __launch_bounds__(1024) void moe_group(const int32_t *ids, int n_pairs, int n_used,
                                                  int n_expert, int32_t *grp_expert,
                                                  int32_t *grp_start, int32_t *grp_count,
                                                  int32_t *sub_start, int32_t *slot_of_pair,
                                                  int32_t *pair_idx, int max_chunks) {
    __shared__ int sub_lds[GROUP_MAX_EXPERTS];
    __shared__ int start_lds[GROUP_MAX_EXPERTS];
    (void)n_used;
    __shared__ int hist[GROUP_MAX_EXPERTS];
    __shared__ int cursor[GROUP_MAX_EXPERTS];
    __shared__ int totals[2];  // chunks, twins
    const int tid = threadIdx.x;
    for (int e = tid; e < n_expert; e += blockDim.x) hist[e] = 0;
    __syncthreads();
    // a pair whose id is outside [0, n_expert) joins no group: its slot is -1,
    // which the chunk quantizers skip and the combine counts as no term
    // ids in batches of PB per thread, all of a batch's loads in flight
    // before its first atomic (one memory round trip per batch, not per id)
    constexpr int PB = 8;
    // the last batch's ids stay in registers for the scatter below (with up
    // to PB * blockDim.x pairs, the only batch: no second round trip)
    int eid[PB];
    int last_base = 0;
    for (int base = 0; base < n_pairs; base += PB * (int)blockDim.x) {
#pragma unroll
        for (int k = 0; k < PB; ++k) {
            const int p = base + k * (int)blockDim.x + tid;
            eid[k] = p < n_pairs ? ids[p] : -1;
        }
#pragma unroll
        for (int k = 0; k < PB; ++k)
            if ((unsigned)eid[k] < (unsigned)n_expert) atomicAdd(&hist[eid[k]], 1);
        last_base = base;
    }
    __syncthreads();
    // exclusive prefix sums over experts (thread e owns expert e) of the
    // pair counts and of the 16-token chunk counts
    __shared__ int wsum_c[GROUP_MAX_EXPERTS / WAVE], wsum_s[GROUP_MAX_EXPERTS / WAVE],
        wsum_t[GROUP_MAX_EXPERTS / WAVE];
    const int lane = tid & 63, wave = tid >> 6;
    const int c = tid < n_expert ? hist[tid] : 0, ch = (c + 15) / 16, tw = (ch + 1) / 2;
    const int ic = wave_incl_sum_i(c), is = wave_incl_sum_i(ch), it = wave_incl_sum_i(tw);
    if (lane == WAVE - 1) {
        wsum_c[wave] = ic;
        wsum_s[wave] = is;
        wsum_t[wave] = it;
    }
    __syncthreads();
    int start = ic - c, sub = is - ch, tst = it - tw;
    for (int w = 0; w < wave; ++w) {
        start += wsum_c[w];
        sub += wsum_s[w];
        tst += wsum_t[w];
    }
    if (tid < n_expert) {
        grp_expert[tid] = tid;
        grp_start[tid] = start;
        grp_count[tid] = c;
        sub_start[tid] = sub;
        sub_start[n_expert + 1 + tid] = tst;
        sub_lds[tid] = sub;
        start_lds[tid] = start;
        cursor[tid] = start;
        if (tid == n_expert - 1) {
            sub_start[n_expert] = sub + ch;
            sub_start[2 * n_expert + 1] = tst + tw;
            totals[0] = sub + ch;
            totals[1] = tst + tw;
        }
        if (max_chunks > 0) {
            GroupItem *sub_info = (GroupItem *)(sub_start + group_items_offset(n_expert));
            GroupItem *twin_info = sub_info + max_chunks;
            for (int j = 0; j < ch; ++j)
                sub_info[sub + j] = GroupItem{tid, j, sub + j, c, start, 0, 0, 0};
            for (int j = 0; j < tw; ++j)
                twin_info[tst + j] = GroupItem{tid, 2 * j, sub + 2 * j, c, start, 2 * j + 1 < ch, 0, 0};
        }
    }
    __syncthreads();
    if (max_chunks > 0) {
        // the records past the last chunk / twin: no work (expert -1), so a
        // wave of the grid's spare items needs no other load to know it
        GroupItem *sub_info = (GroupItem *)(sub_start + group_items_offset(n_expert));
        GroupItem *twin_info = sub_info + max_chunks;
        for (int i = totals[0] + tid; i < max_chunks; i += blockDim.x)
            sub_info[i] = GroupItem{-1, 0, 0, 0, 0, 0, 0, 0};
        for (int i = totals[1] + tid; i < max_chunks; i += blockDim.x)
            twin_info[i] = GroupItem{-1, 0, 0, 0, 0, 0, 0, 0};
    }
    // batches in reverse, the one still in registers first
    for (int base = last_base; base >= 0 && n_pairs > 0; base -= PB * (int)blockDim.x) {
        if (base != last_base) {
#pragma unroll
            for (int k = 0; k < PB; ++k) {
                const int p = base + k * (int)blockDim.x + tid;
                eid[k] = p < n_pairs ? ids[p] : -1;
            }
        }
#pragma unroll
        for (int k = 0; k < PB; ++k) {
            const int p = base + k * (int)blockDim.x + tid;
            if (p >= n_pairs) continue;
            const int e = eid[k];
            if ((unsigned)e >= (unsigned)n_expert) {
                slot_of_pair[p] = -1;
                continue;
            }
            const int pos = atomicAdd(&cursor[e], 1);
            const int j = pos - start_lds[e];
            slot_of_pair[p] = (sub_lds[e] + j / 16) * 16 + j % 16;
            pair_idx[pos] = p;
        }
    }
}

}  // namespace

int launch_moe_group(const int32_t *ids, int n_pairs, int n_used, int n_expert,
                     int32_t *grp_expert, int32_t *grp_start, int32_t *grp_count,
                     int32_t *sub_start, int32_t *slot_of_pair, int32_t *pair_idx,
                     hipStream_t st, int max_chunks) {
    if (n_expert > GROUP_MAX_EXPERTS || n_expert <= 0 || max_chunks < 0) return -1;
    hipLaunchKernelGGL(moe_group, dim3(1), dim3(1024), 0, st, ids, n_pairs, n_used, n_expert,
                       grp_expert, grp_start, grp_count, sub_start, slot_of_pair, pair_idx,
                       max_chunks);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

}  // namespace llamd
