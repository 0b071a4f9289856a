// Replays streamed-layer calls through the library's host policy
// (hummingflight_amd/csrc/expert_stream_policy.h) without a GPU, so the CPU
// tests can compare every decision with the oracle's restatement.
//
// stdin, one command per line:
//   reset SLOTS
//   opt PREFETCH EMA EMA_ALPHA OVERLAP_FLOOR OVERLAP_ALPHA [EXTRA_DEPTH PROB_RESIDENT]
//   call LAYER NEXT K E1 .. EK [P1 .. PK]   (NEXT: 0 no next layer, 1 streamed,
//        2 HBM-resident; P: the winners' routing weights)
//   forget LAYER  (the layer was re-registered: drop its cached experts)
//   drop SLOT     (the copy into SLOT failed: the slot becomes empty)
// stdout per call: "L s0 c0 s1 c1 ..." (slot, copy flag per selected expert),
// then "S e0 s0 e1 s1 ..." (copied-ahead expert and slot); at the end the
// counters in the order of hfmoe_stream_counters.
#include <cstdio>
#include <iostream>
#include <sstream>
#include <string>
#include <vector>

#include "expert_stream_policy.h"

int main() {
    hf::ExpertStreamPolicy p;
    p.reset(16);
    std::string line;
    while (std::getline(std::cin, line)) {
        std::istringstream in(line);
        std::string cmd;
        in >> cmd;
        if (cmd == "reset") {
            int slots = 0;
            in >> slots;
            const hf::StreamPolicyOptions keep = p.opt;
            p.reset(slots);
            p.opt = keep;
        } else if (cmd == "opt") {
            int pf = 0, ema = 0, extra = 0, prob = 0;
            in >> pf >> ema >> p.opt.ema_alpha >> p.opt.overlap_floor >> p.opt.overlap_alpha;
            if (in >> extra >> prob) {
                p.opt.extra_depth = extra;
                p.opt.prob_resident = prob != 0;
            }
            p.opt.prefetch = pf != 0;
            p.opt.ema_predictor = ema != 0;
        } else if (cmd == "drop") {
            int slot = -1;
            in >> slot;
            p.drop_slot(slot);
        } else if (cmd == "forget") {
            int layer = 0;
            in >> layer;
            p.forget_layer(layer);
        } else if (cmd == "call") {
            int layer = 0, next = 0, k = 0;
            in >> layer >> next >> k;
            std::vector<int> topk(k);
            for (int& e : topk) in >> e;
            std::vector<float> probs(k);
            bool have_probs = k > 0;
            for (float& v : probs) have_probs = have_probs && static_cast<bool>(in >> v);
            // The same sequence as streamed_forward_t1 (streamed.hip).
            const std::vector<int> guess =
                p.route_done(layer, topk.data(), have_probs ? probs.data() : nullptr, k, next != 0, next == 1);
            int held[24];
            std::printf("L");
            for (int r = 0; r < k; ++r) {
                bool copy = false;
                held[r] = p.lookup(layer, topk[r], held, r, &copy);
                std::printf(" %d %d", held[r], copy ? 1 : 0);
            }
            std::printf("\nS");
            int nheld = k;
            for (int e : guess) {
                if (e < 0 || nheld >= 24) continue;
                const int s = p.stage(layer + 1, e, held, nheld);
                if (s < 0) continue;
                held[nheld++] = s;
                std::printf(" %d %d", e, s);
            }
            std::printf("\n");
        }
    }
    const hf::StreamPolicyCounters& n = p.n;
    std::printf("C %llu %llu %llu %llu %llu %llu %llu %llu %llu\n", (unsigned long long)n.lookups,
                (unsigned long long)n.hits, (unsigned long long)n.misses, (unsigned long long)n.pred_staged,
                (unsigned long long)n.pred_consumed, (unsigned long long)n.pred_wasted,
                (unsigned long long)n.pred_resident, (unsigned long long)n.copies, (unsigned long long)n.pinned);
    return 0;
}
