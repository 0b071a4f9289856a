// expert_stream_policy.h -- host-side policy of the streamed-expert path.
//
// Two decisions, kept free of HIP so that a plain C++ build can replay them:
//
//  * which HBM slot holds a (layer, expert) weight set.  The slot pool is an
//    LRU cache like the reference's device expert cache
//    (ExpertGpuCache::acquireSlot, src/compute/cuda_backend.cpp:322-363): a
//    free slot first, else the least recently used one.  From the reference's
//    host expert LRU (src/storage/lru_cache.h:137-199) it takes the soft boost
//    (an entry survives `protect` eviction sweeps) and the wasted-prefetch
//    count (a speculatively copied entry evicted before any lookup used it).
//    Slots the current call already uses are never victims: their copies and
//    the kernels reading them are still queued.
//
//  * which experts of layer L+1 to copy ahead once layer L has routed
//    (Scheduler::onLayerRouterDone, src/engine/scheduler.cpp:238-388, with
//    predictNextLayerExperts, :180-219): the previous token's selection at
//    layer L+1, or layer L's own selection when L+1 has none yet.  A layer
//    keeps an EMA of how many winners consecutive tokens share (:247-258);
//    guesses for L+1 are dropped while that EMA is below the floor (:303-306).
//    With the popularity predictor on (setPopularityPredictor, :158-165) each
//    routed expert's heat rolls as heat = a + (1 - a) * heat and the layer's
//    hottest routed expert gets a one-sweep boost (:279-292).  The reference
//    then fills the guess list with hot experts only up to the size of the
//    list it already has, which adds none (:190-218); that is kept.
//
//  * the router-probability mode (Scheduler::setRouterPrefetch,
//    scheduler.cpp:148-156, rules :320-352), given each winner's routing
//    weight: extra_depth adds this token's winners not already guessed, by
//    descending weight, as further layer L+1 copy-aheads (after the overlap
//    gate, so also when it is closed); prob_resident keeps a running maximum
//    of the layer's routing weights and pins a resident winner whose weight is
//    at least 0.9 x that maximum once it has been looked up twice before (a
//    pinned slot is never a victim while an unpinned one is available).
//
// Order of one call, the reference's (moeLayer calls onLayerRouterDone,
// glm_forward.cpp:548, before the expert loop's getExpertPtr, :564, :623):
// route_done (history, heat and boost, pins, guesses), then the demand
// lookups in rank order, then the copy-aheads of the guesses.
#pragma once

#include <algorithm>
#include <cstdint>
#include <map>
#include <unordered_map>
#include <vector>

namespace hf {

struct StreamPolicyOptions {
    bool prefetch = true;          // copy predicted next-layer experts ahead
    bool ema_predictor = false;    // popularity heat + boost of the hottest
    float ema_alpha = 0.1f;        // heat blend, (0, 1]
    float overlap_floor = 0.5f;    // kSpecOverlapFloor (scheduler.cpp:51)
    float overlap_alpha = 0.5f;    // kSpecOverlapAlpha (scheduler.cpp:52)
    int extra_depth = 0;           // prefetchExtraDepth (scheduler.cpp:148-156, 320-336)
    bool prob_resident = false;    // probPriority: probability-weighted residency (:338-352)
};

struct StreamPolicyCounters {
    uint64_t lookups = 0;        // demand lookups (selected experts)
    uint64_t hits = 0;           // ... found resident (or already being copied)
    uint64_t misses = 0;         // ... that needed a copy
    uint64_t pred_staged = 0;    // predicted experts copied ahead (routedPredStaged)
    uint64_t pred_consumed = 0;  // staged entries a demand lookup then used (routedPredConsumed)
    uint64_t pred_wasted = 0;    // staged entries evicted unused (prefetchWasted)
    uint64_t pred_resident = 0;  // predictions already resident: no copy
    uint64_t copies = 0;         // expert weight sets copied host -> HBM
    uint64_t pinned = 0;         // resident experts pinned by the probability rule
};

inline uint64_t expert_key(int layer, int expert) {
    return ((uint64_t)(uint32_t)layer << 32) | (uint32_t)expert;
}

class ExpertStreamPolicy {
public:
    static constexpr uint64_t kEmpty = ~0ull;

    void reset(int slots) {
        key_.assign(slots, kEmpty);
        prev_.assign(slots, -1);
        next_.assign(slots, -1);
        protect_.assign(slots, 0);
        staged_.assign(slots, 0);
        used_.assign(slots, 0);
        pinned_.assign(slots, 0);
        access_.clear();
        max_prob_.clear();
        where_.clear();
        head_ = tail_ = -1;
        last_topk_.clear();
        overlap_.clear();
        heat_.clear();
        n = StreamPolicyCounters{};
    }
    int slots() const { return (int)key_.size(); }
    uint64_t key_of(int slot) const { return key_[slot]; }
    int find(uint64_t key) const {
        auto it = where_.find(key);
        return it == where_.end() ? -1 : it->second;
    }

    // Demand lookup of layer's expert.  Returns the slot; *copy tells whether
    // the weights must be copied into it.  claimed: slots this call already uses.
    int lookup(int layer, int expert, const int* claimed, int nclaimed, bool* copy) {
        const uint64_t k = expert_key(layer, expert);
        ++n.lookups;
        ++access_[k];  // PlacementDirector::recordAccess in getExpertPtr (scheduler.cpp:652)
        int s = find(k);
        if (s >= 0) {
            ++n.hits;
            if (staged_[s] && !used_[s]) ++n.pred_consumed;
            used_[s] = 1;
            touch(s);
            *copy = false;
            return s;
        }
        ++n.misses;
        s = victim(claimed, nclaimed, true);
        place(s, k, false);
        ++n.copies;
        *copy = true;
        return s;
    }

    // Layer finished routing with selection topk[0..k) and the winners'
    // routing weights probs[0..k) (or null).  Updates the routing history,
    // heat and pins, and returns the experts of layer + 1 to stage: empty when
    // there is no next layer (has_next false: the reference stops there,
    // scheduler.cpp:293-294), when prefetch is off or the next layer's experts
    // are not streamed.
    std::vector<int> route_done(int layer, const int* topk, const float* probs, int k, bool has_next,
                                bool next_streamed) {
        std::vector<int> cur(topk, topk + k);
        std::vector<int>& last = last_topk_[layer];
        float& ema = overlap_[layer];
        if (!last.empty() && !cur.empty()) {
            int common = 0;
            for (int e : cur) common += std::find(last.begin(), last.end(), e) != last.end();
            const float frac = (float)common / (float)std::max(last.size(), cur.size());
            ema = opt.overlap_alpha * frac + (1.0f - opt.overlap_alpha) * ema;
        }
        last = cur;
        if (opt.prob_resident && probs) {
            float& mx = max_prob_[layer];
            for (int r = 0; r < k; ++r) mx = std::max(mx, probs[r]);
        }
        if (opt.ema_predictor) {
            const float a = opt.ema_alpha > 0.0f && opt.ema_alpha <= 1.0f ? opt.ema_alpha : 0.1f;
            int best = -1;
            float best_heat = -1.0f;
            for (int e : cur) {
                float& h = heat_[expert_key(layer, e)];
                h = a + (1.0f - a) * h;
                if (h > best_heat) {
                    best_heat = h;
                    best = e;
                }
            }
            if (best >= 0) boost(expert_key(layer, best), 1);
        }
        if (!has_next) return {};
        auto it = last_topk_.find(layer + 1);
        std::vector<int> guess = (it != last_topk_.end() && !it->second.empty()) ? it->second : cur;
        auto ot = overlap_.find(layer + 1);
        if ((ot == overlap_.end() ? 0.0f : ot->second) < opt.overlap_floor) guess.clear();
        if (opt.extra_depth > 0 && probs) {
            // This token's winners by descending weight (ties in rank order),
            // skipping those already guessed.
            std::vector<int> order;
            for (int r = 0; r < k; ++r)
                if (probs[r] > 0.0f && std::find(guess.begin(), guess.end(), topk[r]) == guess.end())
                    order.push_back(r);
            std::stable_sort(order.begin(), order.end(), [&](int a, int b) { return probs[a] > probs[b]; });
            for (int i = 0; i < (int)order.size() && i < opt.extra_depth; ++i) guess.push_back(topk[order[i]]);
        }
        if (opt.prob_resident && probs) {
            const float mx = max_prob_[layer];
            for (int r = 0; mx > 0.0f && r < k; ++r) {
                const uint64_t key = expert_key(layer, topk[r]);
                auto ac = access_.find(key);
                if (probs[r] >= 0.9f * mx && ac != access_.end() && ac->second >= 2) pin(key);
            }
        }
        if (!opt.prefetch || !next_streamed) return {};
        return guess;
    }

    // Copy-ahead of a predicted expert.  Returns the slot to copy into, or -1
    // when it is already resident or every candidate slot is protected.
    int stage(int layer, int expert, const int* claimed, int nclaimed) {
        const uint64_t k = expert_key(layer, expert);
        if (find(k) >= 0) {
            ++n.pred_resident;
            return -1;
        }
        const int s = victim(claimed, nclaimed, false);
        if (s < 0) return -1;
        place(s, k, true);
        ++n.pred_staged;
        ++n.copies;
        return s;
    }

    // Drops every cached expert of `layer` (its weights were re-registered or
    // unregistered) and the layer's routing history.  Slots become empty.
    void forget_layer(int layer) {
        for (int s = 0; s < slots(); ++s) {
            if (key_[s] == kEmpty || (int)(uint32_t)(key_[s] >> 32) != layer) continue;
            where_.erase(key_[s]);
            unlink(s);
            key_[s] = kEmpty;
            protect_[s] = 0;
            staged_[s] = used_[s] = pinned_[s] = 0;
        }
        last_topk_.erase(layer);
        overlap_.erase(layer);
        max_prob_.erase(layer);
        for (auto it = access_.begin(); it != access_.end();)
            it = (int)(uint32_t)(it->first >> 32) == layer ? access_.erase(it) : std::next(it);
        for (auto it = heat_.begin(); it != heat_.end();)
            it = (int)(uint32_t)(it->first >> 32) == layer ? heat_.erase(it) : std::next(it);
    }

    // Empties one slot: the copy meant to fill it was never queued, so the
    // entry placed there must not be served.  A later lookup copies it again.
    void drop_slot(int s) {
        if (s < 0 || s >= slots() || key_[s] == kEmpty) return;
        where_.erase(key_[s]);
        unlink(s);
        key_[s] = kEmpty;
        protect_[s] = 0;
        staged_[s] = used_[s] = pinned_[s] = 0;
    }

    // Pin a resident entry: no victim while an unpinned slot can be taken.
    void pin(uint64_t key) {
        const int s = find(key);
        if (s < 0 || pinned_[s]) return;
        pinned_[s] = 1;
        ++n.pinned;
    }
    bool is_pinned(int slot) const { return pinned_[slot] != 0; }

    // Soft boost: most recent, and survives `cycles` eviction sweeps.
    void boost(uint64_t key, int cycles) {
        const int s = find(key);
        if (s < 0) return;
        protect_[s] = std::max(protect_[s], cycles);
        touch(s);
    }

    StreamPolicyOptions opt;
    StreamPolicyCounters n;

private:
    // Recency list over slots: head_ = most recent, tail_ = least recent.
    void unlink(int s) {
        if (prev_[s] >= 0) next_[prev_[s]] = next_[s]; else if (head_ == s) head_ = next_[s];
        if (next_[s] >= 0) prev_[next_[s]] = prev_[s]; else if (tail_ == s) tail_ = prev_[s];
        prev_[s] = next_[s] = -1;
    }
    void push_front(int s) {
        prev_[s] = -1;
        next_[s] = head_;
        if (head_ >= 0) prev_[head_] = s;
        head_ = s;
        if (tail_ < 0) tail_ = s;
    }
    void touch(int s) {
        unlink(s);
        push_front(s);
    }
    static bool contains(const int* v, int nv, int s) {
        for (int i = 0; i < nv; ++i)
            if (v[i] == s) return true;
        return false;
    }
    // An empty slot (lowest index) first.  Else one sweep from the least
    // recent end: claimed and pinned slots are skipped, a protected one spends
    // one protection and survives, the first other one is the victim.  A
    // demand lookup must get a slot, so when the sweep finds none it takes the
    // least recent unclaimed unpinned slot regardless of protection, and when
    // every unclaimed slot is pinned, the least recent of those (unpinning
    // it: the reference's host cache would serve the expert uncached); a
    // copy-ahead gives up.
    int victim(const int* claimed, int nclaimed, bool must) {
        for (int s = 0; s < slots(); ++s)
            if (key_[s] == kEmpty && !contains(claimed, nclaimed, s)) return s;
        for (int s = tail_; s >= 0; s = prev_[s]) {
            if (contains(claimed, nclaimed, s) || pinned_[s]) continue;
            if (protect_[s] > 0) {
                --protect_[s];
                continue;
            }
            return s;
        }
        if (!must) return -1;
        for (int s = tail_; s >= 0; s = prev_[s])
            if (!contains(claimed, nclaimed, s) && !pinned_[s]) return s;
        for (int s = tail_; s >= 0; s = prev_[s])
            if (!contains(claimed, nclaimed, s)) return s;
        return -1;
    }
    void place(int s, uint64_t k, bool staged) {
        if (key_[s] != kEmpty) {
            if (staged_[s] && !used_[s]) ++n.pred_wasted;
            where_.erase(key_[s]);
            unlink(s);
        }
        key_[s] = k;
        where_[k] = s;
        protect_[s] = 0;
        pinned_[s] = 0;
        staged_[s] = staged;
        used_[s] = !staged;
        push_front(s);
    }

    std::vector<uint64_t> key_;
    std::vector<int> prev_, next_, protect_;
    std::vector<uint8_t> staged_, used_, pinned_;
    std::unordered_map<uint64_t, int> access_;  // demand lookups per (layer, expert)
    std::map<int, float> max_prob_;             // running maximum routing weight per layer
    std::unordered_map<uint64_t, int> where_;
    int head_ = -1, tail_ = -1;
    std::map<int, std::vector<int>> last_topk_;
    std::map<int, float> overlap_;
    std::map<uint64_t, float> heat_;
};

}  // namespace hf
