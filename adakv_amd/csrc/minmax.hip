// Block scores of minmax summaries (Quest's per-block key bounds,
// adakv/estimator.py:50-57,76-79, adakv/attention.py:131-138,190-198): the
// score kernel of score.hpp instantiated for rows [max | min] of 2*head_dim
// elements against [max(q, 0) | min(q, 0)].  Its own translation unit so that
// it compiles in parallel with the centroid instantiation in plan.hip.
#include "score.hpp"

namespace adakv {

hipError_t launch_score_minmax(ScoreArgs& a, int cdt, int D, hipStream_t s) {
  return launch_score_kind<true>(a, cdt, D, s);
}

}  // namespace adakv
