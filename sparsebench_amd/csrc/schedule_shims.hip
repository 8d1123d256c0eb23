// The layer kernels' tile schedules, compiled for the CPU: extern "C" shims
// over the same __host__ __device__ functions the kernels call
// (common.hpp: xcd_remap, split_tail, split_tail_slack, tile_coords;
// expert_chunks.hpp: balanced_chunk_tile, lpt_group_tile, pair_units_per_xcd,
// pair_tile_for), so tests/test_tile_schedules.py checks the compiled
// mappings themselves. Part of the tool library (libsparsebench_probe.so),
// not of libsparsebench_hip.so's C ABI. No kernel runs.

#include "expert_chunks.hpp"

using namespace sb;

extern "C" int sbt_xcd_remap(int bid, int live) { return xcd_remap(bid, live); }

extern "C" void sbt_split_tail(int bid, int tiles, int cus_per_xcd, int* tile, int* half) {
  const TailTile t = split_tail(bid, tiles, cus_per_xcd);
  *tile = t.tile;
  *half = t.half;
}

extern "C" int64_t sbt_split_tail_slack(int cus) { return split_tail_slack(cus); }

extern "C" void sbt_tile_coords(int tile, int live_rb, int slices, int group, int* rb, int* slice) {
  tile_coords(tile, live_rb, slices, group, rb, slice);
}

extern "C" int sbt_balanced_chunk_tile(int bid, int chunks, int slices, int* rank, int* slice) {
  return balanced_chunk_tile(bid, chunks, slices, rank, slice) ? 1 : 0;
}

extern "C" int sbt_pair_units_per_xcd(int units) { return pair_units_per_xcd(units); }

extern "C" int sbt_pair_tile_for(int bid, int pairs, int singles, int slices, int cus, int* single, int* k,
                                 int* slice, int* half) {
  bool s = false;
  const bool ok = pair_tile_for(bid, pairs, singles, slices, cus, &s, k, slice, half);
  *single = s ? 1 : 0;
  return ok ? 1 : 0;
}

extern "C" void sbt_lpt_group_tile(int local, int groups, int slices, uint32_t big, int* pos, int* slice) {
  lpt_group_tile(local, groups, slices, big, pos, slice);
}
