// Stable counting sort of cluster labels (host-side launch interface).
#pragma once

#include "common.hpp"

namespace peco {

// Tokens per sort tile: one tile is ranked by a single wavefront, 64 tokens per step. The
// k-means assign kernel adds its labels to these histograms with atomics.
constexpr int kSortTile = 256;
constexpr int kMaxSortClusters = 16384;

struct SortProblem {
    const int32_t* labels;  // [batch, tokens], values in [0, clusters)
    int32_t* indices;       // [batch, tokens]: original token at each sorted position
    int32_t* ranks;         // nullable [batch, tokens]: sorted position of each token
    int32_t* counts;        // nullable [batch, clusters]
    int32_t* offsets;       // [batch, clusters + 1]: first sorted position of each cluster
    int32_t* tile_hist;     // workspace [batch, tiles, clusters]
    int32_t* next_hist;     // nullable, fused sort only: histograms cleared for the next producer
    int batch, tokens, clusters, tiles;
    int block_begin;        // first linear (batch, tile) block of this problem
    int batch_begin;        // first linear batch entry of this problem (scan grid)
    int group_begin;        // first linear (batch, tile group) workgroup (fused grid)
    int scan_groups;        // groups of kScanTiles tiles per batch entry
    int scan_group_begin;   // first linear (batch, scan group) workgroup (group scan grid)
};

constexpr int kMaxSortProblems = 2;

struct SortArgs {
    SortProblem p[kMaxSortProblems];
    int num;
    int total_blocks;   // sum of batch * tiles
    int total_batches;  // sum of batch
    int zero_hist;      // sort_place clears each consumed tile histogram (for accumulating producers)
    int fused;          // one sort_fused launch instead of scan + place (sort_fusable problems only)
    int total_groups;   // sum of batch * ceil(tiles / kFusedTiles)
    int total_scan_groups;  // sum of batch * scan_groups
};

// Fused sort: a workgroup ranks kFusedTiles consecutive tiles (one per wavefront) and derives
// the cluster offsets of its batch entry from the tile histograms itself. Each workgroup reads
// the whole [tiles, clusters] histogram of its entry, so this is for small entries only.
constexpr int kFusedTiles = 4;
constexpr int kFusedMaxTiles = 32;
constexpr int kFusedMaxClusters = 1024;

inline bool sort_fusable(int tokens, int clusters) {
    return ceil_div(tokens, kSortTile) <= kFusedMaxTiles && clusters <= kFusedMaxClusters;
}

inline int sort_tiles(int tokens) { return static_cast<int>(ceil_div(tokens, kSortTile)); }

// The unfused scan is a reduce-then-scan over groups of kScanTiles tiles: per group, the
// (tile, cluster) counts become exclusive prefixes within the group and the group totals go
// to a second area; per batch entry, the group totals are scanned into cluster offsets and
// group starts; the place kernel adds its group's start to its in-group prefixes.
constexpr int kScanTiles = 32;

inline int sort_scan_groups(int tokens) { return static_cast<int>(ceil_div(sort_tiles(tokens), kScanTiles)); }

// [batch, tiles, clusters] tile histograms followed by [batch, scan groups, clusters] group
// totals.
inline size_t sort_workspace_ints(int batch, int tokens, int clusters) {
    return static_cast<size_t>(batch) * (sort_tiles(tokens) + sort_scan_groups(tokens)) * clusters;
}

// Fills block_begin/batch_begin/totals for problems[0..num).
void sort_args_finalize(SortArgs& args);

// with_hist=false: tile_hist already holds the per-tile label counts (e.g. accumulated
// by the k-means assign kernel), so only the scan and place kernels run (or, with
// args.fused, the single fused kernel, which leaves tile_hist unchanged and clears
// next_hist instead).
hipError_t launch_cluster_sort(const SortArgs& args, hipStream_t stream, bool with_hist);

}  // namespace peco
