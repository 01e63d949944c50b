// staged_plan_test.cpp — the staged mode's slicing (pf_staged.h) on the host
// (no GPU), built by tests/test_native.py from the library's own sources:
//   * a Llama-3-8B prefix load (32 layers of 40 MiB, 64 MiB load slices,
//     128 MiB slots): the first layer in 16 + 24 MiB, every later layer one
//     40 MiB slice; waited for layer by layer, every layer one slice; the
//     same with the first layer left to the kernel; Qwen3-8B and oversized
//     first layers waited for layer by layer;
//   * its save: 128 MiB slices spanning layers, ten of them;
//   * a tensor-parallel rank's load (5 MiB layers): the first two layers
//     alone while slices grow, then seven layers a slice;
//   * empty layers (in place with the slice before them, or with the open
//     one), a layer copied in place in order, a change of chunk size, a
//     chunk larger than the slice, one larger than the slot (an error), and
//     descriptors that start after a kernel's;
//   * 3000 random calls against the rules every cut must keep: each chunk
//     once and in order, one chunk size per slice, a slice within its size
//     (sizes doubling from the first for loads), descriptors contiguous,
//     layers done in order and with the slice that holds their last chunk,
//     and a load's layer ending its slice once the slice is half full.
// Exit status 0 and "ok" on success; the first failed checks are printed.
#include <cstdio>
#include <random>
#include <string>
#include <vector>

#include "pf_staged.h"

using namespace pf;

namespace {

int failures = 0;

void expect(bool cond, const std::string& what) {
  if (!cond && ++failures <= 20) std::printf("FAILED: %s\n", what.c_str());
}

constexpr uint64_t MiB = 1ull << 20;

// A layer of n chunks of cb bytes; addresses are (layer, index) codes so
// every chunk is told apart.
LayerPlan layer(uint32_t li, size_t n, uint64_t cb, bool ordered = false) {
  LayerPlan p;
  p.chunk_bytes = cb;
  p.ordered = ordered;
  for (size_t i = 0; i < n; ++i) p.chunks.push_back({(uint64_t(li) << 32) | i, i});
  return p;
}

uint64_t step_bytes(const StagedStep& st) { return st.n_chunks * st.chunk_bytes; }

// Slices of a call planned as the transfer code does: layers [0, head) then
// [head, n), each range cut; with a kernel head, only [head, n).
struct Call {
  std::vector<LayerPlan> plans;
  StagedPlan sp;
  int rc = PF_OK;
};

Call plan(std::vector<LayerPlan> plans, uint64_t slot, uint64_t slice, bool is_save,
          uint32_t head, bool kernel_head = false, size_t desc_start = 0,
          uint64_t first_layer = 0) {
  Call c;
  c.plans = std::move(plans);
  const uint32_t n = static_cast<uint32_t>(c.plans.size());
  StagedPlanner pl(slot, slice, is_save, n, &c.sp);
  if (first_layer) pl.start_with_layer(first_layer);
  if (!kernel_head) {
    if ((c.rc = pl.add(c.plans, 0, head)) != PF_OK) return c;
    if ((c.rc = pl.cut()) != PF_OK) return c;
  } else {
    pl.start_descriptors_at(desc_start);
  }
  if (head < n) {
    if ((c.rc = pl.add(c.plans, head, n)) != PF_OK) return c;
    c.rc = pl.cut();
  }
  return c;
}

std::string sizes(const StagedPlan& sp) {
  std::string s;
  for (const StagedStep& st : sp.steps)
    s += (st.ordered_layer >= 0 ? "o" : std::to_string(step_bytes(st) / MiB)) + " ";
  return s;
}

// The layers each step touches, as "first-last".
std::string spans(const StagedPlan& sp) {
  std::string s;
  for (const StagedStep& st : sp.steps) {
    if (st.ordered_layer >= 0) {
      s += "o" + std::to_string(st.ordered_layer) + " ";
      continue;
    }
    const uint32_t a = sp.pieces[st.piece_begin].layer, b = sp.pieces[st.piece_end - 1].layer;
    s += std::to_string(a) + (a == b ? "" : "-" + std::to_string(b)) + " ";
  }
  return s;
}

// Every rule a cut must keep (loads: slice sizes double from the first).
void check_rules(const Call& c, uint64_t slot, uint64_t slice, bool is_save, uint32_t head,
                 bool kernel_head, size_t desc_start, const std::string& what,
                 uint64_t first_layer = 0) {
  const StagedPlan& sp = c.sp;
  const uint64_t max_cap = std::min(slot, slice);
  uint64_t cap = is_save ? max_cap : std::max<uint64_t>(1, std::min(16 * MiB, max_cap / 4));
  if (!is_save) cap = std::max(cap, std::min(max_cap, first_layer));
  const uint32_t first = kernel_head ? head : 0;
  // Each chunk once, in order: walk the pieces against the plans.
  uint32_t li = first;
  size_t ci = 0;
  auto skip_done = [&]() {
    while (li < c.plans.size() && (c.plans[li].ordered || ci == c.plans[li].chunks.size())) {
      ++li;
      ci = 0;
    }
  };
  size_t desc = desc_start;
  std::vector<int64_t> last_step(c.plans.size(), -2);
  for (size_t si = 0; si < sp.steps.size(); ++si) {
    const StagedStep& st = sp.steps[si];
    const std::string at = what + " step " + std::to_string(si);
    if (st.ordered_layer >= 0) {
      expect(st.piece_begin == st.piece_end, at + ": pieces in an in-place step");
      expect(c.plans[static_cast<size_t>(st.ordered_layer)].ordered, at + ": not an ordered layer");
      last_step[static_cast<size_t>(st.ordered_layer)] = static_cast<int64_t>(si);
      continue;
    }
    expect(st.piece_end > st.piece_begin && st.n_chunks > 0, at + ": empty slice");
    expect(st.desc_first == desc, at + ": descriptors not contiguous");
    desc += st.n_chunks;
    const uint64_t bytes = step_bytes(st);
    expect(bytes <= std::max(cap, st.chunk_bytes), at + ": " + std::to_string(bytes) +
                                                       " bytes past the slice size " +
                                                       std::to_string(cap));
    expect(bytes <= slot, at + ": larger than a slot");
    uint64_t acc = 0;
    size_t n = 0;
    for (size_t k = st.piece_begin; k < st.piece_end; ++k) {
      const Piece& p = sp.pieces[k];
      skip_done();
      expect(p.layer == li && p.begin == ci && p.end > p.begin, at + ": chunks out of order");
      if (p.layer != li || p.begin != ci) return;
      expect(c.plans[li].chunk_bytes == st.chunk_bytes, at + ": mixed chunk sizes");
      ci = p.end;
      n += p.end - p.begin;
      acc += (p.end - p.begin) * st.chunk_bytes;
      last_step[li] = static_cast<int64_t>(si);
      const bool layer_end = ci == c.plans[li].chunks.size();
      // A load's slice holds a layer end inside it only while less than
      // half full at the largest slice size.
      if (!is_save && layer_end && k + 1 < st.piece_end)
        expect(cap == max_cap && 2 * acc < cap, at + ": a load slice continued past a layer "
                                                    "end once half full");
    }
    expect(n == st.n_chunks, at + ": chunk count");
    // A slice stops early only at a layer end (loads), a change of chunk
    // size, an in-place step, or the end of a planned range.
    const Piece& lastp = sp.pieces[st.piece_end - 1];
    const bool ends_layer = lastp.end == c.plans[lastp.layer].chunks.size();
    const bool full = bytes + st.chunk_bytes > std::max(cap, st.chunk_bytes);
    if (!full && !ends_layer) expect(false, at + ": slice cut inside a layer before full");
    if (!full && ends_layer && is_save && si + 1 < sp.steps.size()) {
      const StagedStep& nx = sp.steps[si + 1];
      const bool range_end = !kernel_head && lastp.layer + 1 == head;
      bool gap_ordered = nx.ordered_layer >= 0;
      for (uint32_t l = lastp.layer + 1; l < c.plans.size() && !gap_ordered; ++l) {
        if (c.plans[l].ordered) gap_ordered = true;
        if (!c.plans[l].chunks.empty()) break;
      }
      expect(range_end || gap_ordered || nx.chunk_bytes != st.chunk_bytes,
             at + ": save slice closed before full");
    }
    cap = std::min(max_cap, 2 * cap);
  }
  skip_done();
  expect(li == c.plans.size(), what + ": chunks left unsliced");
  expect(sp.n_desc == desc, what + ": n_desc");
  // Layers done in order, with the slice holding their last chunk; an empty
  // layer with the slice before it.
  int64_t prev = -1;
  for (size_t l = 0; l < c.plans.size(); ++l) {
    const int64_t d = sp.done_at[l];
    const std::string at = what + " layer " + std::to_string(l);
    if (l < first) {
      expect(d == kNotSliced, at + ": a kernel layer sliced");
      continue;
    }
    expect(d >= prev && d < static_cast<int64_t>(sp.steps.size()), at + ": done_at " +
                                                                        std::to_string(d));
    if (last_step[l] != -2) expect(d == last_step[l], at + ": not done with its last slice");
    prev = d;
  }
}

}  // namespace

int main() {
  const uint64_t slot = 128 * MiB;
  // Llama-3-8B prefix: 32 layers, K and V of 640 blocks, 32 KiB each.
  auto llama = [](uint32_t layers, uint64_t layer_bytes) {
    std::vector<LayerPlan> v;
    for (uint32_t l = 0; l < layers; ++l) v.push_back(layer(l, layer_bytes / (32 << 10), 32 << 10));
    return v;
  };
  {
    const Call c = plan(llama(32, 40 * MiB), slot, 64 * MiB, false, 1);
    expect(c.rc == PF_OK, "llama load");
    std::string want = "16 24 ";
    for (int l = 1; l < 32; ++l) want += "40 ";
    expect(sizes(c.sp) == want, "llama load slices: " + sizes(c.sp));
    expect(c.sp.done_at[0] == 1 && c.sp.done_at[31] == 32, "llama load done_at");
    check_rules(c, slot, 64 * MiB, false, 1, false, 0, "llama load");
  }
  {
    // Waited for layer by layer: the first layer one slice of its own.
    const Call c = plan(llama(32, 40 * MiB), slot, 64 * MiB, false, 1, false, 0, 40 * MiB);
    std::string want;
    for (int l = 0; l < 32; ++l) want += "40 ";
    expect(c.rc == PF_OK && sizes(c.sp) == want, "llama layered load: " + sizes(c.sp));
    expect(c.sp.done_at[0] == 0 && c.sp.done_at[31] == 31, "llama layered load done_at");
    check_rules(c, slot, 64 * MiB, false, 1, false, 0, "llama layered load", 40 * MiB);
    // Qwen3-8B's 313 blocks (19.56 MiB layers): the first two layers alone
    // while slices grow, then two layers a slice.
    const uint64_t q = 313 * 2 * (32 << 10);
    const Call qw = plan(llama(36, q), slot, 64 * MiB, false, 1, false, 0, q);
    expect(qw.rc == PF_OK && spans(qw.sp).rfind("0 1 2-3 4-5 ", 0) == 0,
           "qwen3 layered load: " + spans(qw.sp));
    check_rules(qw, slot, 64 * MiB, false, 1, false, 0, "qwen3 layered load", q);
    // A first layer larger than the largest slice: slices of that size.
    const Call big = plan(llama(4, 100 * MiB), slot, 64 * MiB, false, 1, false, 0, 100 * MiB);
    expect(big.rc == PF_OK && sizes(big.sp).rfind("64 36 64 36 ", 0) == 0,
           "large-layer layered load: " + sizes(big.sp));
    check_rules(big, slot, 64 * MiB, false, 1, false, 0, "large-layer layered load", 100 * MiB);
  }
  {
    const Call c = plan(llama(32, 40 * MiB), slot, 64 * MiB, false, 1, true, 40);
    std::string want = "16 24 ";
    for (int l = 2; l < 32; ++l) want += "40 ";
    expect(c.rc == PF_OK && sizes(c.sp) == want, "llama kernel-head load: " + sizes(c.sp));
    expect(c.sp.steps[0].desc_first == 40, "kernel-head descriptors");
    check_rules(c, slot, 64 * MiB, false, 1, true, 40, "llama kernel-head load");
  }
  {
    const Call c = plan(llama(32, 40 * MiB), slot, 128 * MiB, true, 32);
    std::string want;
    for (int s = 0; s < 10; ++s) want += "128 ";
    expect(c.rc == PF_OK && sizes(c.sp) == want, "llama save slices: " + sizes(c.sp));
    for (uint32_t l = 0; l < 32; ++l)
      expect(c.sp.done_at[l] == static_cast<int64_t>(((l + 1) * 40 - 1) / 128),
             "llama save done_at of layer " + std::to_string(l));
    check_rules(c, slot, 128 * MiB, true, 32, false, 0, "llama save");
  }
  {
    const Call c = plan(llama(32, 5 * MiB), slot, 64 * MiB, false, 1);
    expect(c.rc == PF_OK && spans(c.sp) == "0 1 2-8 9-15 16-22 23-29 30-31 ",
           "tp load slices: " + spans(c.sp));
    check_rules(c, slot, 64 * MiB, false, 1, false, 0, "tp load");
  }
  {
    // Empty layers: first (before any slice), after a closed slice, inside
    // an open one; an in-place layer; a chunk size change.
    std::vector<LayerPlan> v;
    v.push_back(layer(0, 0, 4096));
    v.push_back(layer(1, 10, 4096));
    v.push_back(layer(2, 0, 4096));
    v.push_back(layer(3, 10, 4096));
    v.push_back(layer(4, 0, 4096));
    v.push_back(layer(5, 4, 4096, true));
    v.push_back(layer(6, 10, 8192));
    v.push_back(layer(7, 10, 4096));
    const Call save = plan(v, slot, 128 * MiB, true, 8);
    expect(save.rc == PF_OK && spans(save.sp) == "1-3 o5 6 7 ", "mixed save: " + spans(save.sp));
    const std::vector<int64_t> want_save = {-1, 0, 0, 0, 0, 1, 2, 3};
    expect(save.sp.done_at == want_save, "mixed save done_at");
    check_rules(save, slot, 128 * MiB, true, 8, false, 0, "mixed save");
    const Call load = plan(v, slot, 64 * MiB, false, 8);
    // Loads close each layer while slices grow.
    expect(load.rc == PF_OK && spans(load.sp) == "1 3 o5 6 7 ", "mixed load: " + spans(load.sp));
    const std::vector<int64_t> want_load = {-1, 0, 0, 1, 1, 2, 3, 4};
    expect(load.sp.done_at == want_load, "mixed load done_at");
    check_rules(load, slot, 64 * MiB, false, 8, false, 0, "mixed load");
  }
  {
    // A chunk larger than the slice fills a slice alone; one larger than
    // the slot is refused.
    std::vector<LayerPlan> v{layer(0, 3, 48 * MiB)};
    const Call c = plan(v, slot, 32 * MiB, true, 1);
    expect(c.rc == PF_OK && sizes(c.sp) == "48 48 48 ", "big chunks: " + sizes(c.sp));
    check_rules(c, slot, 32 * MiB, true, 1, false, 0, "big chunks");
    std::vector<LayerPlan> w{layer(0, 1, slot + 256)};
    const Call d = plan(w, slot, 64 * MiB, false, 1);
    expect(d.rc == PF_ERR_INVALID_ARGUMENT, "a chunk larger than the slot is refused");
  }
  // Random calls.
  std::mt19937_64 rng(20261202);
  const uint64_t sizes_b[] = {512, 4096, 32768, 65536, 1 << 20};
  for (int t = 0; t < 3000 && failures == 0; ++t) {
    const bool is_save = rng() % 2;
    const uint32_t n = 1 + rng() % 40;
    const uint64_t cb0 = sizes_b[rng() % 5];
    std::vector<LayerPlan> v;
    for (uint32_t l = 0; l < n; ++l) {
      const uint64_t cb = rng() % 6 == 0 ? sizes_b[rng() % 5] : cb0;
      const size_t cnt = rng() % 7 == 0 ? 0 : rng() % 400;
      v.push_back(layer(l, cnt, cb, !is_save && rng() % 15 == 0));
    }
    const uint64_t slot_t = (1 + rng() % 64) * 256 * 1024;  // 256 KiB .. 16 MiB
    const uint64_t slice_t = (1 + rng() % 64) * 128 * 1024;
    const uint32_t head = is_save ? n : 1 + static_cast<uint32_t>(rng() % n);
    const bool kh = !is_save && head < n && rng() % 3 == 0;
    const size_t ds = kh ? rng() % 500 : 0;
    bool too_big = false;
    for (uint32_t l = kh ? head : 0; l < n; ++l)
      too_big = too_big || (!v[l].ordered && !v[l].chunks.empty() && v[l].chunk_bytes > slot_t);
    // A load waited for layer by layer starts with its first layer's bytes
    // (as the transfer code passes them: the first non-empty layer copied
    // through the staging).
    uint64_t first = 0;
    if (!is_save && !kh && rng() % 2 == 0)
      for (uint32_t l = 0; l < head && first == 0; ++l)
        if (!v[l].ordered && !v[l].chunks.empty()) first = v[l].chunks.size() * v[l].chunk_bytes;
    const Call c = plan(v, slot_t, slice_t, is_save, head, kh, ds, first);
    const std::string what = "random call " + std::to_string(t);
    if (too_big) {
      expect(c.rc == PF_ERR_INVALID_ARGUMENT, what + ": oversized chunk accepted");
      continue;
    }
    expect(c.rc == PF_OK, what + ": refused");
    if (c.rc == PF_OK) check_rules(c, slot_t, slice_t, is_save, head, kh, ds, what, first);
  }
  if (failures) return 1;
  std::printf("ok\n");
  return 0;
}
