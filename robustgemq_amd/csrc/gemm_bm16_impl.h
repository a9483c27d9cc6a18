// 16-row (decode) launches of the grouped GEMM, shared by the gemm_bm16*.hip
// units: each instantiates launch16 for some activation / output types, so
// the largest set of kernel variants compiles in parallel units.
#pragma once

#include "gemm_impl.h"

namespace moeq {

template <int ADT, int ODT, bool SILU>
int launch16(const GemmArgs &g, int max_tiles, int splits, hipStream_t s) {
  // Few column blocks (small decode batches) or a long K range: split K over
  // the waves of 16-column blocks instead, so enough waves keep weight
  // fetches in flight and no wave walks a long chain of chunks.
  using S = Shape<16, SILU>;
  const int64_t col_blocks = int64_t(max_tiles) * cdiv(g.N, tile_cols<S, false>());
  const int chunks = int(cdiv(g.nchunks, splits));
  // tiles of at most 16 rows (a batch of at most 16 tokens: a token picks an
  // expert at most once) run the kernel without the two-block path, whose
  // extra code costs every launch a fixed ~0.4 us
  const bool one = g.max_rows > 0 && g.max_rows <= 16;
  // Tall tiles (the caller expects 12+ rows per expert, e.g. 64 tokens over 8
  // experts): every wave reloads its activation fragments per chunk, so
  // twice the columns per wave halve those loads per weight byte (Mixtral
  // B = 64: 271 -> 232 us per layer); with fewer rows the extra columns cost
  // more waves in flight than they save (B = 1..32 slower).
  constexpr int NBW = 2 * S::NB;
  const bool wide = !one && g.rows_hint >= 12;
  if (col_blocks < 256 || chunks > 32)
    return one ? launch_one<16, SILU, ADT, ODT, true, false>(g, max_tiles, splits, s)
         : wide ? launch_one<16, SILU, ADT, ODT, true, true, NBW>(g, max_tiles, splits, s)
                : launch_one<16, SILU, ADT, ODT, true, true>(g, max_tiles, splits, s);
  return one ? launch_one<16, SILU, ADT, ODT, false, false>(g, max_tiles, splits, s)
       : wide ? launch_one<16, SILU, ADT, ODT, false, true, NBW>(g, max_tiles, splits, s)
              : launch_one<16, SILU, ADT, ODT, false, true>(g, max_tiles, splits, s);
}

}  // namespace moeq
