// pf_staged.h — a layer's chunk plan, and the staged mode's cutting of a
// call's chunks into slices (pf_transfer.cpp), in a header of their own so
// the slicing rules are tested on the host (tests/native/staged_plan_test.cpp).
#pragma once

#include <algorithm>
#include <climits>
#include <cstddef>
#include <cstdint>
#include <vector>

#include "pf_common.h"

namespace pf {

// ---------------------------------------------------------------------------
// Chunk planning.  A layer's transfer is a list of equal-size chunks, each
// pairing a device address inside the paged layer tensor with an address on
// the other side (host pinned memory, or any device-visible buffer).
// ---------------------------------------------------------------------------
struct Chunk {
  uint64_t dev;   // address inside the layer tensor
  uint64_t host;  // address on the host (or staging) side
};

struct LayerPlan {
  uint64_t chunk_bytes = 0;
  std::vector<Chunk> chunks;
  // The reference merges the K list and the V list of a split layer in two
  // separate batch_copy_segments_to_gpu calls (gpu_worker.rs:242-256); runs
  // never cross this index.
  size_t list_break = 0;
  // True when the chunks must be copied one after another in list order to
  // reproduce the reference's result (needs_order in pf_transfer.cpp).
  bool ordered = false;
};

struct Piece {
  uint32_t layer;
  size_t begin, end;  // chunks [begin, end) of the layer's plan
};

struct StagedStep {
  size_t piece_begin = 0, piece_end = 0;  // pieces[piece_begin, piece_end)
  uint64_t chunk_bytes = 0;
  size_t n_chunks = 0;
  size_t desc_first = 0;
  int64_t ordered_layer = -1;  // >= 0: this step is that layer's in-place copies
  int lane = 0;
};

struct StagedPlan {
  std::vector<StagedStep> steps;
  std::vector<Piece> pieces;
  // Per layer: the step after which its bytes are in place (-1: before any).
  std::vector<int64_t> done_at;
  size_t n_desc = 0;
};

// A load's first slice is a quarter of the load slice size, at most 16 MiB;
// later slices double up to the load slice size.  Each copy-engine command
// costs about 11 us besides its bytes (80 x 16 MiB host-to-device copies on
// one engine moved 55.5 GB/s, 20 x 64 MiB 57.0), so slices grow to amortize
// it while the first layer lands early (the Llama prefix's 40 MiB first
// layer is two copies, 16 + 24 MiB).
constexpr uint64_t kStagedLoadFirstSlice = 16ull << 20;

// done_at of a layer not sliced yet.
constexpr int64_t kNotSliced = INT64_MIN;

// Cuts the chunks of a call's layers into slices, in layer order, a range of
// layers at a time (a pipelined load slices its first layer, queues its
// copies, and slices the rest while they run).  Plans are indexed by the
// call's layer numbers.
class StagedPlanner {
 public:
  // slot_bytes: one staging slot; slice_bytes: the direction's largest slice.
  StagedPlanner(uint64_t slot_bytes, uint64_t slice_bytes, bool is_save, size_t num_layers,
                StagedPlan* sp)
      : sp_(sp),
        is_save_(is_save),
        slot_bytes_(slot_bytes),
        max_cap_(std::min(slot_bytes, slice_bytes)) {
    cap_ = is_save ? max_cap_
                   : std::max<uint64_t>(1, std::min(kStagedLoadFirstSlice, max_cap_ / 4));
    sp_->steps.clear();
    sp_->pieces.clear();
    sp_->done_at.assign(num_layers, kNotSliced);
    sp_->n_desc = 0;
  }

  // Slices layers [begin, end), after those sliced so far.
  int add(const std::vector<LayerPlan>& plans, uint32_t begin, uint32_t end) {
    for (uint32_t li = begin; li < end; ++li) {
      const LayerPlan& p = plans[li];
      if (p.ordered) {
        close();
        StagedStep st;
        st.piece_begin = st.piece_end = sp_->pieces.size();
        st.ordered_layer = li;
        sp_->steps.push_back(st);
        sp_->done_at[li] = static_cast<int64_t>(sp_->steps.size()) - 1;
        continue;
      }
      if (p.chunks.empty()) {
        // In place once everything before it is: after the open slice, if any.
        sp_->done_at[li] = static_cast<int64_t>(sp_->steps.size()) - (cur_.n_chunks > 0 ? 0 : 1);
        continue;
      }
      if (p.chunk_bytes > slot_bytes_)
        return fail(PF_ERR_INVALID_ARGUMENT,
                    strf("staging slot (%llu bytes) smaller than one chunk (%llu)",
                         (unsigned long long)slot_bytes_, (unsigned long long)p.chunk_bytes));
      if (cur_.n_chunks > 0 && cur_.chunk_bytes != p.chunk_bytes) close();
      size_t i = 0;
      while (i < p.chunks.size()) {
        // A slice holds at least one chunk, even one larger than the slice size.
        const uint64_t lcap = std::max(cap_, p.chunk_bytes);
        const size_t room = static_cast<size_t>((lcap - cur_bytes_) / p.chunk_bytes);
        if (room == 0) {
          close();
          continue;
        }
        const size_t take = std::min(room, p.chunks.size() - i);
        cur_.chunk_bytes = p.chunk_bytes;
        sp_->pieces.push_back({li, i, i + take});
        cur_.n_chunks += take;
        cur_bytes_ += take * p.chunk_bytes;
        i += take;
      }
      sp_->done_at[li] = static_cast<int64_t>(sp_->steps.size());  // the open slice
      // A load's layer ends its last slice while slices still grow (its
      // first layers) and once that slice is half full, so the layer lands
      // without waiting for the next one's bytes.
      if (!is_save_ && (cap_ < max_cap_ || 2 * cur_bytes_ >= cap_)) close();
    }
    return PF_OK;
  }

  // A load waited for layer by layer starts with a slice that holds its
  // first layer whole (up to the largest slice size): that layer is then one
  // copy and one scatter, and each kernel on the way to it can wait for a
  // whole kernel of other work holding every CU (a GEMM whose workgroups
  // fill the register files).  Later slices double from there.  Before any
  // layer is added.
  void start_with_layer(uint64_t bytes) {
    if (!is_save_ && sp_->steps.empty() && cur_.n_chunks == 0)
      cap_ = std::max(cap_, std::min(max_cap_, bytes));
  }

  // Descriptors of the slices start at index n (before any slice).
  void start_descriptors_at(size_t n) { sp_->n_desc = n; }

  // The largest slice this planner makes of chunks up to `chunk` bytes: the
  // slice cap, or one chunk when a chunk is larger.
  uint64_t max_slice_bytes(uint64_t chunk) const { return std::max(max_cap_, chunk); }

  // Closes the open slice: the steps so far are final.
  int cut() {
    close();
    if (sp_->n_desc > 0xffffffffull) return fail(PF_ERR_INVALID_ARGUMENT, "too many chunks");
    return PF_OK;
  }

 private:
  void close() {
    if (cur_.n_chunks > 0) {
      cur_.piece_end = sp_->pieces.size();
      cur_.desc_first = sp_->n_desc;
      sp_->n_desc += cur_.n_chunks;
      sp_->steps.push_back(cur_);
      cap_ = std::min(max_cap_, 2 * cap_);
    }
    cur_ = StagedStep{};
    cur_.piece_begin = sp_->pieces.size();
    cur_bytes_ = 0;
  }

  StagedPlan* sp_;
  bool is_save_;
  uint64_t slot_bytes_, max_cap_, cap_ = 0, cur_bytes_ = 0;
  StagedStep cur_;
};

}  // namespace pf
