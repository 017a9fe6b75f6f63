// Host-side check of the prefill job planner (place_prefill_jobs in
// q38_attn.cpp, compiled into this program): for prompts of 1..4096 tokens
// after prefixes of 0..16,773,120 (the longest sequence the cache accepts is
// 16,777,216 tokens, so key-block indices pass 65535), every (head pair, query block) job's key blocks
// are covered exactly once by its pieces, a piece starts on a block that
// every row of its job sees whole, partial slots are unique and dense, the
// split list matches the pieces, and no bin holds more than the table allows.
// Prints the worst bin load against the average and exits non-zero on the
// first violation.
#include "../../qwen3.8_27b_in_rust_amd/csrc/host/q38_attn.cpp"

// The device scratch lookup lives in a hipcc-built object; the planner never
// reaches it, so this program answers for it with an error.
int q38_scratch_address(int, void **ptr) {
    *ptr = nullptr;
    return -1;
}
#include <cassert>
#include <map>
int main() {
    int cases = 0, worst_case_ratio_x100 = 0;
    for (int base : {0, 1, 31, 32, 100, 1000, 3000, 3001, 9000, 50000, 131000, 2097088, 2097120, 2100000,
                     16773120}) {
        for (int T : {1, 2, 17, 63, 64, 65, 200, 512, 700, 1000, 1024, 1500, 2048, 3000, 4096}) {
            const int nq = (T + 63) / 64;
            q38_prefill_job table[Q38_PREFILL_BINS * Q38_PREFILL_JOBS_MAX];
            q38_prefill_split splits[Q38_PREFILL_SPLITS_MAX];
            int ns = -1, nslots = -1;
            const int per = place_prefill_jobs(base, T, nq, table, splits, &ns, &nslots);
            if (per < 1 || per > Q38_PREFILL_JOBS_MAX) { printf("bad per %d base %d T %d: %s\n", per, base, T, q38_last_error()); return 1; }
            std::map<int, std::vector<std::pair<int, int>>> cover; // code -> pieces (kb0, kb1)
            std::map<int, int> slot_use;
            long maxload = 0, total = 0;
            for (int b = 0; b < Q38_PREFILL_BINS; ++b) {
                long load = 0;
                bool ended = false;
                for (int i = 0; i < per; ++i) {
                    const q38_prefill_job &j = table[b * per + i];
                    if (j.code == 0xFFFF) { ended = true; continue; }
                    if (ended) { printf("job after end marker\n"); return 1; }
                    const int qb = j.code & 63, hp = j.code >> 6;
                    if (qb >= nq || hp >= 3 || j.kb1 <= j.kb0) { printf("bad job\n"); return 1; }
                    const int q_last = std::min((qb + 1) * 64, T) - 1;
                    const int n_kb = (base + q_last) / 32 + 1;
                    if (j.kb1 > n_kb) { printf("piece past the job's blocks\n"); return 1; }
                    const int first_pos = base + qb * 64;
                    if (j.kb0 > 0 && j.kb0 * 32 + 31 > first_pos) { printf("piece start not seen whole: base %d T %d qb %d kb0 %d\n", base, T, qb, j.kb0); return 1; }
                    if (j.slot != 0xFFFF) {
                        if (j.slot >= nslots || slot_use[j.slot]++) { printf("bad/dup slot\n"); return 1; }
                    } else if (j.kb0 != 0 || j.kb1 != n_kb) { printf("whole job with a partial range\n"); return 1; }
                    cover[j.code].push_back({j.kb0, j.kb1});
                    load += j.kb1 - j.kb0;
                }
                maxload = std::max(maxload, load);
                total += load;
            }
            if ((int)cover.size() != 3 * nq) { printf("jobs missing: %zu of %d\n", cover.size(), 3 * nq); return 1; }
            for (auto &kv : cover) {
                auto v = kv.second;
                std::sort(v.begin(), v.end());
                const int qb = kv.first & 63;
                const int n_kb = (base + std::min((qb + 1) * 64, T) - 1) / 32 + 1;
                int at = 0;
                for (auto &p : v) { if (p.first != at) { printf("gap/overlap\n"); return 1; } at = p.second; }
                if (at != n_kb) { printf("not covered\n"); return 1; }
            }
            // splits list: each split job's slots are its pieces
            int pieces = 0;
            for (int g = 0; g < ns; ++g) {
                auto &v = cover[splits[g].code];
                if ((int)v.size() != splits[g].n) { printf("split count mismatch\n"); return 1; }
                pieces += splits[g].n;
            }
            if (pieces != nslots || (int)slot_use.size() != nslots) { printf("slot count mismatch\n"); return 1; }
            const long avg = (total + 63) / 64;
            worst_case_ratio_x100 = std::max<int>(worst_case_ratio_x100, (int)(100 * maxload / std::max<long>(avg, 1)));
            ++cases;
        }
    }
    printf("%d cases ok; worst max/avg bin load %.2f\n", cases, worst_case_ratio_x100 / 100.0);
    return 0;
}
