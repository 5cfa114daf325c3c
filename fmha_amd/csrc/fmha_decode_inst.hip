// fmha_decode_inst.hip -- explicit instantiations of the launchers declared
// in fmha_decode_launch.hpp, one slice per compilation: fmha_amd/_build.py
// compiles this file once for each FMHA_DECODE_PART in [0, FMHA_DECODE_PARTS)
// and links the objects with fmha_decode_api.hip.  Part 0 holds the kernels
// every long-row path shares (the split-KV statistics and combine passes, query-group
// padding); every other part instantiates launchers, and with them kernels,
// that no other part does.
//
// FMHA_DECODE_PARTS 63
#ifndef FMHA_DECODE_PART
#error "compile with -DFMHA_DECODE_PART=<part>"
#endif
#define FMHA_DECODE_INSTANTIATING
#if FMHA_DECODE_PART == 0
#define FMHA_DECODE_SHARED_KERNELS
#endif
#include "fmha_decode_launch.hpp"

namespace fmha_decode {
namespace host {

#if FMHA_DECODE_PART == 0

// The statistics pass of split-KV: the global max and sum per (batch, query
// head).  One lane per head for rows of at most 16 blocks, else one
// workgroup per head sized to the row's block count (8 blocks per thread
// and round).
void launch_split_stats(const SplitArgs& a, hipStream_t stream) {
  const uint32_t heads = (uint32_t)a.batch * (uint32_t)a.num_heads_q;
  if (a.nblk <= 16)
    hipLaunchKernelGGL(fmha_decode::splitkv_stats_lane_kernel, dim3((heads + 255) / 256), dim3(256), 0, stream, a);
  else if (a.nblk <= 8 * 64)
    hipLaunchKernelGGL(fmha_decode::splitkv_stats_kernel<64>, dim3(heads), dim3(64), 0, stream, a);
  else if (a.nblk <= 8 * 256)
    hipLaunchKernelGGL(fmha_decode::splitkv_stats_kernel<256>, dim3(heads), dim3(256), 0, stream, a);
  else
    hipLaunchKernelGGL(fmha_decode::splitkv_stats_kernel<1024>, dim3(heads), dim3(1024), 0, stream, a);
}

// The combine pass of split-KV (more than one chunk per row): partial
// outputs summed in chunk order, one lane per 8 dims for few chunks, else a
// workgroup per (head, 32 dims).
template <int D>
void launch_split_combine_d(const SplitArgs& a, hipStream_t stream) {
  const uint32_t heads = (uint32_t)a.batch * (uint32_t)a.num_heads_q;
  if (a.nchunks <= 16) {
    const uint64_t lanes = (uint64_t)heads * (D / 8);
    hipLaunchKernelGGL(fmha_decode::splitkv_combine_kernel<D>, dim3((unsigned)((lanes + 255) / 256)), dim3(256), 0,
                       stream, a);
  } else if (a.nchunks <= 256) {
    hipLaunchKernelGGL((fmha_decode::splitkv_combine_block_kernel<D, 256>), dim3(heads * (D / 32)), dim3(256), 0,
                       stream, a);
  } else {
    hipLaunchKernelGGL((fmha_decode::splitkv_combine_block_kernel<D, 1024>), dim3(heads * (D / 32)), dim3(1024), 0,
                       stream, a);
  }
}

void launch_split_combine(const SplitArgs& a, int d, hipStream_t stream) {
  switch (d) {
    case 64: return launch_split_combine_d<64>(a, stream);
    case 128: return launch_split_combine_d<128>(a, stream);
    default: return launch_split_combine_d<256>(a, stream);
  }
}

hipError_t launch_pad_query_group(const uint16_t* q, uint16_t* qp, uint64_t streams, int G, int GP, int D,
                                  hipStream_t stream) {
  plan_note("pad_query_group(G=%d to %d)", G, GP);
  const uint64_t chunks = streams * (uint64_t)GP * (uint64_t)(D / 8);
  hipLaunchKernelGGL(pad_query_group_kernel, dim3((uint32_t)((chunks + kPadThreads - 1) / kPadThreads)),
                     dim3(kPadThreads), 0, stream, q, qp, streams, G, 0, G, GP, D);
  return hipGetLastError();
}

hipError_t launch_unpad_output_group(const uint16_t* op, uint16_t* o, uint64_t streams, int G, int GP, int D,
                                     hipStream_t stream) {
  const uint64_t chunks = streams * (uint64_t)G * (uint64_t)(D / 8);
  hipLaunchKernelGGL(unpad_output_group_kernel, dim3((uint32_t)((chunks + kPadThreads - 1) / kPadThreads)),
                     dim3(kPadThreads), 0, stream, op, o, streams, G, 0, G, GP, D);
  return hipGetLastError();
}

#elif FMHA_DECODE_PART == 1
template hipError_t launch_group<64, kLayoutPacked, false>(const DecodeArgs&, int, int, int, hipStream_t);
#elif FMHA_DECODE_PART == 2
template hipError_t launch_group<64, kLayoutPacked, true>(const DecodeArgs&, int, int, int, hipStream_t);
#elif FMHA_DECODE_PART == 3
template hipError_t launch_group<64, kLayoutStrided, false>(const DecodeArgs&, int, int, int, hipStream_t);
#elif FMHA_DECODE_PART == 4
template hipError_t launch_group<64, kLayoutPaged, false>(const DecodeArgs&, int, int, int, hipStream_t);
#elif FMHA_DECODE_PART == 5
template hipError_t launch_group<128, kLayoutPacked, false>(const DecodeArgs&, int, int, int, hipStream_t);
#elif FMHA_DECODE_PART == 6
template hipError_t launch_group<128, kLayoutPacked, true>(const DecodeArgs&, int, int, int, hipStream_t);
#elif FMHA_DECODE_PART == 7
template hipError_t launch_group<128, kLayoutStrided, false>(const DecodeArgs&, int, int, int, hipStream_t);
#elif FMHA_DECODE_PART == 8
template hipError_t launch_group<128, kLayoutPaged, false>(const DecodeArgs&, int, int, int, hipStream_t);
#elif FMHA_DECODE_PART == 9
template hipError_t launch_group<256, kLayoutPacked, false>(const DecodeArgs&, int, int, int, hipStream_t);
#elif FMHA_DECODE_PART == 10
template hipError_t launch_group<256, kLayoutPacked, true>(const DecodeArgs&, int, int, int, hipStream_t);
#elif FMHA_DECODE_PART == 11
template hipError_t launch_group<256, kLayoutStrided, false>(const DecodeArgs&, int, int, int, hipStream_t);
#elif FMHA_DECODE_PART == 12
template hipError_t launch_group<256, kLayoutPaged, false>(const DecodeArgs&, int, int, int, hipStream_t);
#elif FMHA_DECODE_PART == 13
template hipError_t launch_multi<kLayoutPacked, false>(const DecodeArgs&, int, int, int, hipStream_t);
#elif FMHA_DECODE_PART == 14
template hipError_t launch_multi<kLayoutPacked, true>(const DecodeArgs&, int, int, int, hipStream_t);
#elif FMHA_DECODE_PART == 15
template hipError_t launch_multi<kLayoutStrided, false>(const DecodeArgs&, int, int, int, hipStream_t);
#elif FMHA_DECODE_PART == 16
template hipError_t launch_multi<kLayoutPaged, false>(const DecodeArgs&, int, int, int, hipStream_t);
#elif FMHA_DECODE_PART == 17
template hipError_t launch_mfma_d<64, kLayoutPacked>(const GroupArgs&, int, int, hipStream_t);
#elif FMHA_DECODE_PART == 18
template hipError_t launch_mfma_d<64, kLayoutStrided>(const GroupArgs&, int, int, hipStream_t);
#elif FMHA_DECODE_PART == 19
template hipError_t launch_mfma_d<128, kLayoutPacked>(const GroupArgs&, int, int, hipStream_t);
#elif FMHA_DECODE_PART == 20
template hipError_t launch_mfma_d<128, kLayoutStrided>(const GroupArgs&, int, int, hipStream_t);
#elif FMHA_DECODE_PART == 21
template hipError_t launch_mfma_d<256, kLayoutPacked>(const GroupArgs&, int, int, hipStream_t);
#elif FMHA_DECODE_PART == 22
template hipError_t launch_mfma_d<256, kLayoutStrided>(const GroupArgs&, int, int, hipStream_t);
#elif FMHA_DECODE_PART == 23
template hipError_t launch_split_d<64, kLayoutPacked>(const SplitArgs&, int, hipStream_t, bool);
#elif FMHA_DECODE_PART == 24
template hipError_t launch_split_d<64, kLayoutStrided>(const SplitArgs&, int, hipStream_t, bool);
#elif FMHA_DECODE_PART == 25
template hipError_t launch_split_d<64, kLayoutPaged>(const SplitArgs&, int, hipStream_t, bool);
#elif FMHA_DECODE_PART == 26
template hipError_t launch_split_d<64, kLayoutPagedLanes>(const SplitArgs&, int, hipStream_t, bool);
#elif FMHA_DECODE_PART == 27
template hipError_t launch_split_d<64, kLayoutPagedBlock>(const SplitArgs&, int, hipStream_t, bool);
#elif FMHA_DECODE_PART == 28
template hipError_t launch_split_d<64, kLayoutPagedBlockLanes>(const SplitArgs&, int, hipStream_t, bool);
#elif FMHA_DECODE_PART == 29
template hipError_t launch_split_d<128, kLayoutPacked>(const SplitArgs&, int, hipStream_t, bool);
#elif FMHA_DECODE_PART == 30
template hipError_t launch_split_d<128, kLayoutStrided>(const SplitArgs&, int, hipStream_t, bool);
#elif FMHA_DECODE_PART == 31
template hipError_t launch_split_d<128, kLayoutPaged>(const SplitArgs&, int, hipStream_t, bool);
#elif FMHA_DECODE_PART == 32
template hipError_t launch_split_d<128, kLayoutPagedLanes>(const SplitArgs&, int, hipStream_t, bool);
#elif FMHA_DECODE_PART == 33
template hipError_t launch_split_d<128, kLayoutPagedBlock>(const SplitArgs&, int, hipStream_t, bool);
#elif FMHA_DECODE_PART == 34
template hipError_t launch_split_d<128, kLayoutPagedBlockLanes>(const SplitArgs&, int, hipStream_t, bool);
#elif FMHA_DECODE_PART == 35
template hipError_t launch_split_d<256, kLayoutPacked>(const SplitArgs&, int, hipStream_t, bool);
#elif FMHA_DECODE_PART == 36
template hipError_t launch_split_d<256, kLayoutStrided>(const SplitArgs&, int, hipStream_t, bool);
#elif FMHA_DECODE_PART == 37
template hipError_t launch_split_d<256, kLayoutPaged>(const SplitArgs&, int, hipStream_t, bool);
template hipError_t launch_split_d<256, kLayoutPagedLanes>(const SplitArgs&, int, hipStream_t, bool);
#elif FMHA_DECODE_PART == 38
template hipError_t launch_split_d<256, kLayoutPagedBlock>(const SplitArgs&, int, hipStream_t, bool);
template hipError_t launch_split_d<256, kLayoutPagedBlockLanes>(const SplitArgs&, int, hipStream_t, bool);
#elif FMHA_DECODE_PART == 39
template hipError_t launch_split_group_d<64, kLayoutPacked>(const SplitArgs&, hipStream_t);
#elif FMHA_DECODE_PART == 40
template hipError_t launch_split_group_d<64, kLayoutStrided>(const SplitArgs&, hipStream_t);
#elif FMHA_DECODE_PART == 41
template hipError_t launch_split_group_d<64, kLayoutPaged>(const SplitArgs&, hipStream_t);
#elif FMHA_DECODE_PART == 42
template hipError_t launch_split_group_d<64, kLayoutPagedBlock>(const SplitArgs&, hipStream_t);
#elif FMHA_DECODE_PART == 43
template hipError_t launch_split_group_d<128, kLayoutPacked>(const SplitArgs&, hipStream_t);
#elif FMHA_DECODE_PART == 44
template hipError_t launch_split_group_d<128, kLayoutStrided>(const SplitArgs&, hipStream_t);
#elif FMHA_DECODE_PART == 45
template hipError_t launch_split_group_d<128, kLayoutPaged>(const SplitArgs&, hipStream_t);
#elif FMHA_DECODE_PART == 46
template hipError_t launch_split_group_d<128, kLayoutPagedBlock>(const SplitArgs&, hipStream_t);
#elif FMHA_DECODE_PART == 47
template hipError_t launch_split_group_d<256, kLayoutPacked>(const SplitArgs&, hipStream_t);
#elif FMHA_DECODE_PART == 48
template hipError_t launch_split_group_d<256, kLayoutStrided>(const SplitArgs&, hipStream_t);
#elif FMHA_DECODE_PART == 49
template hipError_t launch_split_group_d<256, kLayoutPaged>(const SplitArgs&, hipStream_t);
#elif FMHA_DECODE_PART == 50
template hipError_t launch_split_group_d<256, kLayoutPagedBlock>(const SplitArgs&, hipStream_t);
#elif FMHA_DECODE_PART == 51
template hipError_t launch_exact<64, 1>(const DecodeArgs&, bool, int, int, hipStream_t);
#elif FMHA_DECODE_PART == 52
template hipError_t launch_exact<64, 2>(const DecodeArgs&, bool, int, int, hipStream_t);
#elif FMHA_DECODE_PART == 53
template hipError_t launch_exact<64, 4>(const DecodeArgs&, bool, int, int, hipStream_t);
#elif FMHA_DECODE_PART == 54
template hipError_t launch_exact<64, 8>(const DecodeArgs&, bool, int, int, hipStream_t);
#elif FMHA_DECODE_PART == 55
template hipError_t launch_exact<128, 1>(const DecodeArgs&, bool, int, int, hipStream_t);
#elif FMHA_DECODE_PART == 56
template hipError_t launch_exact<128, 2>(const DecodeArgs&, bool, int, int, hipStream_t);
#elif FMHA_DECODE_PART == 57
template hipError_t launch_exact<128, 4>(const DecodeArgs&, bool, int, int, hipStream_t);
#elif FMHA_DECODE_PART == 58
template hipError_t launch_exact<128, 8>(const DecodeArgs&, bool, int, int, hipStream_t);
#elif FMHA_DECODE_PART == 59
template hipError_t launch_exact<256, 1>(const DecodeArgs&, bool, int, int, hipStream_t);
#elif FMHA_DECODE_PART == 60
template hipError_t launch_exact<256, 2>(const DecodeArgs&, bool, int, int, hipStream_t);
#elif FMHA_DECODE_PART == 61
template hipError_t launch_exact<256, 4>(const DecodeArgs&, bool, int, int, hipStream_t);
#elif FMHA_DECODE_PART == 62
template hipError_t launch_exact<256, 8>(const DecodeArgs&, bool, int, int, hipStream_t);
#else
#error "FMHA_DECODE_PART out of range"
#endif

}  // namespace host
}  // namespace fmha_decode
