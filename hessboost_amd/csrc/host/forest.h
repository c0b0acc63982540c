// A forest resident on one device for batch prediction (the reference's
// GpuModel, src/backend/cuda/predict.rs:401-520).
#pragma once
#include <cstdint>
#include <mutex>
#include <vector>

#include "../abi.h"
#include "hessboost_rocm.h"
#include "runtime.h"

namespace hbr {

class Forest {
public:
    Forest(int ordinal, const hbr_forest_desc &fd);
    std::mutex mu;
    bool failed = false;
    Device &dev() { return dev_; }
    uint32_t n_outputs() const { return n_outputs_; }
    uint64_t n_trees() const { return n_trees_; }
    // x, out, leaf_out, init: device pointers; init (n x n_outputs starting
    // margins) may be null: the base scores.
    void predict_device(const float *x, uint64_t n, uint64_t n_cols, float missing, float *out, int32_t *leaf_out,
                        const float *init = nullptr);
    // The same with x, init and out in host memory (pageable): beyond two
    // chunks of rows, through Device::host_rows (the walk runs on each chunk
    // while the next is staged and copied).
    void predict_host(const float *x, uint64_t n, uint64_t n_cols, float missing, float *out, const float *init);

private:
    Device &dev_;
    uint64_t n_trees_ = 0;
    uint32_t n_outputs_ = 1;
    uint32_t max_feature_ = 0;
    DBuf<uint32_t> value_, meta_, left_, root_, output_;
    DBuf<PredNode> nodes_;
    // compact nodes for the chunked walk (absent when a feature id or a
    // child offset does not fit the compact record)
    bool compact_ok_ = false;
    bool has_categorical_ = false;
    DBuf<uint32_t> categories_, cat_end_;  // the category pool; per node the end of its range
    DBuf<CompactNode> compact_;
    std::vector<uint32_t> tree_nodes_;  // nodes per tree
    uint32_t largest_tree_ = 0;
    // chunk tables for the last LDS capacity used
    uint32_t chunk_cap_ = 0, n_chunks_ = 0;
    DBuf<uint32_t> chunk_tree_, chunk_node_;
    void plan_chunks(uint32_t cap);
    DBuf<int32_t> orig_;
    DBuf<float> weight_, base_;
    // the mirror arena (absent with categorical splits, a non-finite
    // threshold, a feature id of 2^16 - 1 or more, or a child beyond 2^15 - 1
    // nodes of its parent)
    bool mirror_ok_ = false;
    DBuf<MirrorNode> mirror_;
    DBuf<uint32_t> mirror_root_;
    DBuf<int32_t> mirror_orig_;
    DBuf<uint8_t> tree_depth_;
    void build_mirror(const hbr_forest_desc &fd);
    // the pair layout (PredictArgs::pairs): absent unless every split is
    // numeric with a finite threshold on a feature below 127, and the
    // complete trees stay small
    bool pairs_ok_ = false;
    uint32_t pair_levels_ = 0;
    DBuf<PairRecord> pairs_;
    DBuf<uint32_t> pair_values_;
    DBuf<int32_t> pair_orig_;
    void build_pairs(const hbr_forest_desc &fd);
};

}  // namespace hbr
