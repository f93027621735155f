// veckern_bench: the benchmark driver with the reference's command line (bench/bench_main.cpp:24-64) and CSV
// schema (:241-242), over the MI355X search path.
//
//   veckern_bench --n 1000000 --d 128 --m 16 --nq 1000 --k 10            (synthetic Gaussian mixture)
//   veckern_bench --base sift_base.fvecs --query sift_query.fvecs --gt sift_groundtruth.ivecs --m 16
//   veckern_bench --n 10000000 --variants v7,v8 --queries-per-block 4 --label sweep
//
// Differences from the reference driver: the default data is the seeded Gaussian mixture of the headline
// configuration (1000 components, sigma 0.3; --data latent selects the latent-structure source, --data codes
// draws uniform codes and N(0,1) codebooks directly), PQ training defaults to 25 iterations on 50k vectors, the
// default Q is 4, and the CPU reference row is not produced here: the CPU search is test infrastructure in this
// build, timed beside the GPU by bench.py (--cpu-queries is accepted and reported as skipped).
#include <algorithm>
#include <cstdio>
#include <fstream>
#include <memory>
#include <map>
#include <sstream>
#include <string>
#include <vector>

#include "veckern/eval.hpp"
#include "veckern/gpu.hpp"
#include "veckern/io.hpp"
#include "veckern/pq.hpp"

using namespace veckern;

namespace {

struct Options {
    std::size_t n = 1'000'000, d = 128, m = 16, nq = 1000, k = 10, clusters = 1000, seed = 1, latent_dim = 16;
    std::size_t train = 50'000, iters = 25, reps = 5, eval_queries = 100, cpu_queries = 0, rerank = 0;
    std::size_t threads = 256, blocks_per_query = 0, queries_per_block = 4, ilp = 4;
    double sigma = 0.3;
    std::string base, query, gt, csv = "results.csv", variants = "all", label = "default", data = "mixture";
};

void usage() {
    std::puts(
        "data:     --n --d --seed --data mixture|latent|codes --clusters --sigma --latent-dim\n"
        "          | --base X.fvecs|X.bvecs --query X.fvecs|X.bvecs [--gt X.ivecs]\n"
        "search:   --m --nq --k --rerank R\n"
        "training: --train --iters\n"
        "measure:  --reps --eval-queries (0 = skip recall) --cpu-queries (accepted; CPU timing is in bench.py)\n"
        "gpu:      --variants all|v0,...,v8  --threads T  --blocks-per-query B  --queries-per-block Q  --ilp 1|2|4\n"
        "output:   --csv out.csv  --label name");
}

Options parse(int argc, char** argv) {
    Options o;
    const std::map<std::string, std::size_t*> sizes = {
        {"--n", &o.n}, {"--d", &o.d}, {"--m", &o.m}, {"--nq", &o.nq}, {"--k", &o.k}, {"--clusters", &o.clusters},
        {"--seed", &o.seed}, {"--latent-dim", &o.latent_dim}, {"--train", &o.train}, {"--iters", &o.iters},
        {"--reps", &o.reps}, {"--eval-queries", &o.eval_queries}, {"--cpu-queries", &o.cpu_queries},
        {"--rerank", &o.rerank}, {"--threads", &o.threads}, {"--blocks-per-query", &o.blocks_per_query},
        {"--queries-per-block", &o.queries_per_block}, {"--ilp", &o.ilp}};
    const std::map<std::string, std::string*> texts = {{"--base", &o.base}, {"--query", &o.query}, {"--gt", &o.gt},
                                                       {"--csv", &o.csv}, {"--variants", &o.variants},
                                                       {"--label", &o.label}, {"--data", &o.data}};
    for (int i = 1; i < argc; ++i) {
        const std::string flag = argv[i];
        if (flag == "-h" || flag == "--help") {
            usage();
            std::exit(0);
        }
        check(i + 1 < argc, "missing value for " + flag);
        const std::string value = argv[++i];
        if (auto s = sizes.find(flag); s != sizes.end()) *s->second = std::stoull(value);
        else if (auto t = texts.find(flag); t != texts.end()) *t->second = value;
        else if (flag == "--sigma") o.sigma = std::stod(value);
        else throw std::runtime_error("unknown option " + flag + " (try --help)");
    }
    return o;
}

std::vector<float> load_vectors(const std::string& path, std::size_t& n, std::size_t& d, std::size_t max_n) {
    const bool bytes = path.size() > 6 && path.compare(path.size() - 6, 6, ".bvecs") == 0;
    return bytes ? read_bvecs(path, n, d, max_n) : read_fvecs(path, n, d, max_n);
}

double median(std::vector<double> v) {
    std::sort(v.begin(), v.end());
    return v[v.size() / 2];
}

// --variants: "all", or a comma list of prefixes such as "v2,v8" or full names.
bool wanted(const std::string& list, const std::string& name) {
    if (list == "all") return true;
    std::stringstream ss(list);
    for (std::string item; std::getline(ss, item, ',');)
        if (!item.empty() && name.compare(0, item.size(), item) == 0) return true;
    return false;
}

struct Row {
    std::string variant;
    gpu::PQSearcher::LaunchShape shape;
    double lut_ms = 0, scan_ms = 0, select_ms = 0, transfer_ms = 0, total_ms = 0, qps = 0, code_gbs = 0, recall = -1;
};

}  // namespace

int main(int argc, char** argv) try {
    Options o = parse(argc, argv);
    check(o.k >= 1 && o.k <= 128, "--k must be in [1, 128]");

    // ---- data
    Timer data_timer;
    std::vector<float> base, queries, codebook;
    std::vector<uint8_t> codes;
    if (!o.base.empty()) {
        check(!o.query.empty(), "--base requires --query");
        base = load_vectors(o.base, o.n, o.d, o.n);
        std::size_t qd = 0;
        queries = load_vectors(o.query, o.nq, qd, o.nq);
        check(qd == o.d, "query and base dimensions differ");
    } else if (o.data == "codes") {
        check(o.d % o.m == 0, "d must be a multiple of m");
        codes.resize(o.n * o.m);
        uniform_codes(0, o.n, o.m, o.seed, codes.data());
        codebook.resize(o.m * kSubCentroids * (o.d / o.m));
        normal_values(o.seed, 30, 0, codebook.size(), codebook.data());
        queries.resize(o.nq * o.d);
        normal_values(o.seed, 31, 0, queries.size(), queries.data());
        o.eval_queries = 0;  // no base vectors: no exact ground truth
    } else {
        base.resize(o.n * o.d);
        queries.resize(o.nq * o.d);
        const std::size_t query_row = std::size_t(1) << 40;  // queries: a disjoint row range of the same source
        if (o.data == "latent") {
            SyntheticSource src(o.d, o.clusters, o.seed, o.latent_dim);
            src.fill(0, o.n, base.data());
            src.fill(query_row, o.nq, queries.data());
        } else {
            check(o.data == "mixture", "--data must be mixture, latent or codes");
            GaussianMixture src(o.d, o.clusters, static_cast<float>(o.sigma), o.seed);
            src.fill(0, o.n, base.data());
            src.fill(query_row, o.nq, queries.data());
        }
    }
    o.eval_queries = std::min(o.eval_queries, o.nq);
    std::printf("data: n=%zu d=%zu nq=%zu (%s, %.1f s) | PQ m=%zu (%zu B/vector) | k=%zu\n", o.n, o.d, o.nq,
                o.base.empty() ? o.data.c_str() : "files", data_timer.ms() / 1e3, o.m, o.m, o.k);

    // ---- PQ training and encoding (or the directly drawn codebook)
    Timer train_timer;
    ProductQuantizer pq(o.d, o.m);
    if (codes.empty()) {
        pq.train(base.data(), std::min(o.train, o.n), o.iters, o.seed);
        codes.resize(o.n * o.m);
        pq.encode(base.data(), o.n, codes.data());
    } else {
        pq.set_centroids(codebook);
    }
    std::printf("PQ train+encode: %.1f s\n", train_timer.ms() / 1e3);

    // ---- ground truth for the first eval_queries queries
    std::vector<int32_t> truth;
    std::size_t truth_stride = o.k;
    if (o.eval_queries > 0) {
        if (!o.gt.empty()) {
            std::size_t gn = 0;
            truth = read_ivecs(o.gt, gn, truth_stride, o.nq);
            check(gn >= o.eval_queries && truth_stride >= o.k, "ground truth too small");
        } else {
            Timer gt_timer;
            std::vector<Neighbor> exact(o.eval_queries * o.k);
            exact_knn(base.data(), o.n, queries.data(), o.eval_queries, o.d, o.k, exact.data());
            truth.resize(exact.size());
            for (std::size_t j = 0; j < exact.size(); ++j) truth[j] = exact[j].id;
            std::printf("exact ground truth (%zu queries): %.1f s\n", o.eval_queries, gt_timer.ms() / 1e3);
        }
    }
    const std::size_t k_search = o.rerank ? std::max(o.k, o.rerank) : o.k;
    // With --rerank R the search returns R candidates and the GPU re-scores them exactly (gpu::Reranker, results
    // identical to the reference's CPU rerank_exact); the base vectors go to the device once.
    std::unique_ptr<gpu::Reranker> reranker;
    if (o.rerank) {
        check(!base.empty(), "--rerank needs base vectors (not available with --data codes)");
        reranker = std::make_unique<gpu::Reranker>(base.data(), o.n, o.d);
    }
    auto recall_of = [&](const std::vector<Neighbor>& res) -> double {
        if (o.eval_queries == 0) return -1;
        if (o.rerank == 0) return recall_at_k(res.data(), k_search, truth.data(), truth_stride, o.eval_queries, o.k);
        std::vector<Neighbor> rr(o.eval_queries * o.k);
        reranker->rerank(queries.data(), o.eval_queries, res.data(), k_search, o.k, rr.data());
        return recall_at_k(rr.data(), o.k, truth.data(), truth_stride, o.eval_queries, o.k);
    };
    const double code_bytes = static_cast<double>(o.n) * o.m;  // logical PQ code bytes scanned per query
    if (o.cpu_queries > 0)
        std::puts("(--cpu-queries: the CPU reference is timed by bench.py's cpu_baseline leg, not by this driver)");

    // ---- GPU variants
    const auto info = gpu::device_info();
    std::printf("GPU: %s, %d CUs, %.0f GB/s theoretical HBM peak, %zu B LDS per block\n", info.name.c_str(),
                info.sm_count, info.peak_bandwidth_gbs, info.max_smem_per_block);
    gpu::PQSearcher searcher(pq, codes.data(), o.n);
    gpu::Tuning tuning;
    tuning.scan_threads = static_cast<int>(o.threads);
    tuning.blocks_per_query = static_cast<int>(o.blocks_per_query);
    tuning.queries_per_block = static_cast<int>(o.queries_per_block);
    tuning.vectors_per_step = static_cast<int>(o.ilp);
    searcher.set_tuning(tuning);

    std::vector<Row> rows;
    using gpu::ScanVariant;
    for (int vi = 0; vi <= static_cast<int>(ScanVariant::FusedWarpF16); ++vi) {
        const auto v = static_cast<ScanVariant>(vi);
        const std::string name = gpu::variant_name(v);
        if (!wanted(o.variants, name)) continue;
        const bool needs16 = v == ScanVariant::SharedLutVec || v == ScanVariant::FusedVec ||
                             v == ScanVariant::FusedVecMQ || v == ScanVariant::FusedWarp ||
                             v == ScanVariant::FusedWarpF16;
        if (needs16 && o.m % 16 != 0) continue;
        if (v == ScanVariant::Fused) {
            std::printf("%s: not launched in this build (its scratch-resident per-thread list faulted the GPU); "
                        "skipped\n", name.c_str());
            continue;
        }
        std::vector<Neighbor> res(o.nq * k_search);
        searcher.search(queries.data(), o.nq, k_search, v, res.data());  // warm-up and layout build
        std::vector<double> lut, scan, sel, xfer, total;
        for (std::size_t r = 0; r < o.reps; ++r) {
            const auto t = searcher.search(queries.data(), o.nq, k_search, v, res.data());
            lut.push_back(t.lut_ms);
            scan.push_back(t.scan_ms);
            sel.push_back(t.select_ms);
            xfer.push_back(t.transfer_ms);
            total.push_back(t.total_ms());
        }
        Row row;
        row.variant = name;
        row.shape = searcher.last_launch();
        row.lut_ms = median(lut);
        row.scan_ms = median(scan);
        row.select_ms = median(sel);
        row.transfer_ms = median(xfer);
        row.total_ms = median(total);
        row.qps = o.nq / (row.total_ms / 1e3);
        row.code_gbs = code_bytes * o.nq / (row.scan_ms / 1e3) / 1e9;
        if (reranker) {  // the exact re-rank of the whole batch, timed apart from the search (not in the CSV row)
            std::vector<Neighbor> rr(o.nq * o.k);
            std::vector<double> rerank_ms;
            for (std::size_t r = 0; r <= o.reps; ++r) {
                const auto t = reranker->rerank(queries.data(), o.nq, res.data(), k_search, o.k, rr.data());
                if (r > 0) rerank_ms.push_back(t.scan_ms);
            }
            std::printf("%s: GPU exact re-rank of %zu x %zu candidates to k=%zu: %.3f ms kernel\n", name.c_str(), o.nq,
                        k_search, o.k, median(rerank_ms));
        }
        res.resize(std::max<std::size_t>(o.eval_queries, 1) * k_search);
        row.recall = recall_of(res);
        rows.push_back(row);
    }

    // ---- report
    std::printf("\n%-18s %5s %5s %5s %2s %3s %5s %8s %8s %8s %8s %9s %10s %9s %7s\n", "variant", "T", "bx", "gy", "Q",
                "ILP", "waves", "lut ms", "scan ms", "sel ms", "xfer ms", "total ms", "QPS", "code GB/s", "recall");
    for (const auto& r : rows)
        std::printf("%-18s %5d %5d %5d %2d %3d %5.2f %8.3f %8.3f %8.3f %8.3f %9.3f %10.0f %9.1f %7.3f\n",
                    r.variant.c_str(), r.shape.threads, r.shape.blocks_x, r.shape.grid_y, r.shape.queries_per_block,
                    r.shape.vectors_per_step, r.shape.waves, r.lut_ms, r.scan_ms, r.select_ms, r.transfer_ms,
                    r.total_ms, r.qps, r.code_gbs, r.recall);
    std::puts("code GB/s = logical PQ code bytes per query x queries / scan time; it counts L2 and MALL hits");

    const bool exists = std::ifstream(o.csv).good();
    std::ofstream csv(o.csv, std::ios::app);
    if (!exists)
        csv << "label,variant,n,d,m,nq,k,rerank,threads,blocks_x,grid_y,qpb,ilp,blocks_per_sm,waves,lut_ms,scan_ms,"
               "select_ms,transfer_ms,total_ms,qps,code_gbs,recall\n";
    for (const auto& r : rows)
        csv << o.label << ',' << r.variant << ',' << o.n << ',' << o.d << ',' << o.m << ',' << o.nq << ',' << o.k << ','
            << o.rerank << ',' << r.shape.threads << ',' << r.shape.blocks_x << ',' << r.shape.grid_y << ','
            << r.shape.queries_per_block << ',' << r.shape.vectors_per_step << ',' << r.shape.blocks_per_sm << ','
            << r.shape.waves << ',' << r.lut_ms << ',' << r.scan_ms << ',' << r.select_ms << ',' << r.transfer_ms
            << ',' << r.total_ms << ',' << r.qps << ',' << r.code_gbs << ',' << r.recall << '\n';
    std::printf("appended %zu rows to %s\n", rows.size(), o.csv.c_str());
    return 0;
} catch (const std::exception& e) {
    std::fprintf(stderr, "error: %s\n", e.what());
    return 1;
}
