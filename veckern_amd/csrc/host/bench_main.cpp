// veckern_bench: the benchmark driver, a drop-in for the reference's (bench/bench_main.cpp). Its interface is kept:
// the flags and their defaults (:24-27), `--variants` prefix selection (:76-83), the table and the CSV schema
// (:241-242) with one row per variant and a "cpu_reference" row for `--cpu-queries` queries (:155-169), so scripts
// that drive or parse the reference's bench keep working. The driver itself is this build's:
//
//   settings   one flag table (name -> parser) over a Settings struct holding the reference's defaults
//   dataset    synthetic rows (the reference's latent-structure source by default; the Gaussian mixture or directly
//              drawn codes on request) or .fvecs/.bvecs/.ivecs files
//   index      PQ training on the first `--train` rows and encoding, or the drawn codebook and codes
//   scoring    exact ground truth for the first `--eval-queries` queries and recall@k of any result rows, after an
//              exact GPU re-rank when `--rerank R` asks the search for R candidates
//   rows       the CPU search path (veckern/cpu_ref.hpp, all host threads) on the first `--cpu-queries` queries,
//              then each selected GPU variant: one untimed call, `--reps` timed calls, per-stage medians
//   report     the table on stdout, the rows appended to `--csv`
//
//   veckern_bench --n 1000000 --d 128 --m 16 --nq 1000 --k 10
//   veckern_bench --data mixture --clusters 1000 --sigma 0.3 --train 50000 --iters 25 --queries-per-block 4
//   veckern_bench --base sift_base.fvecs --query sift_query.fvecs --gt sift_groundtruth.ivecs --m 16
#include <unistd.h>

#include <algorithm>
#include <cstdio>
#include <fstream>
#include <functional>
#include <memory>
#include <sstream>
#include <stdexcept>
#include <string>
#include <vector>

#ifdef _OPENMP
#include <omp.h>
#endif

#include "veckern/cpu_ref.hpp"
#include "veckern/gpu.hpp"
#include "veckern/io.hpp"

using namespace veckern;

namespace {

// ------------------------------------------------------------------------------------------------ settings

struct Settings {
    // the reference's defaults (bench_main.cpp:24-27)
    std::size_t n = 1'000'000, d = 128, m = 16, nq = 1000, k = 10, clusters = 100, seed = 1, latent_dim = 16;
    std::size_t train = 100'000, iters = 15, reps = 5, eval_queries = 100, cpu_queries = 100, rerank = 0;
    std::size_t threads = 256, blocks_per_query = 0, queries_per_block = 2, ilp = 4;
    std::string base, query, gt, csv = "results.csv", variants = "all", label = "default";
    // this build's additions: the data source and the mixture's spread
    std::string data = "latent";
    double sigma = 0.3;
};

struct Flag {
    const char* name;
    std::function<void(const std::string&)> set;
};

std::vector<Flag> flag_table(Settings& s) {
    auto count = [](std::size_t& field) { return [&field](const std::string& v) { field = std::stoull(v); }; };
    auto text = [](std::string& field) { return [&field](const std::string& v) { field = v; }; };
    return {
        {"--n", count(s.n)}, {"--d", count(s.d)}, {"--m", count(s.m)}, {"--nq", count(s.nq)}, {"--k", count(s.k)},
        {"--clusters", count(s.clusters)}, {"--seed", count(s.seed)}, {"--latent-dim", count(s.latent_dim)},
        {"--train", count(s.train)}, {"--iters", count(s.iters)}, {"--reps", count(s.reps)},
        {"--eval-queries", count(s.eval_queries)}, {"--cpu-queries", count(s.cpu_queries)},
        {"--rerank", count(s.rerank)}, {"--threads", count(s.threads)},
        {"--blocks-per-query", count(s.blocks_per_query)}, {"--queries-per-block", count(s.queries_per_block)},
        {"--ilp", count(s.ilp)}, {"--base", text(s.base)}, {"--query", text(s.query)}, {"--gt", text(s.gt)},
        {"--csv", text(s.csv)}, {"--variants", text(s.variants)}, {"--label", text(s.label)},
        {"--data", text(s.data)}, {"--sigma", [&s](const std::string& v) { s.sigma = std::stod(v); }},
    };
}

const char* kUsage =
    "data:     --n --d --clusters --latent-dim --seed | --base X.fvecs|X.bvecs --query X.fvecs|X.bvecs [--gt X.ivecs]\n"
    "          --data latent|mixture|codes (default latent; mixture: N(0,1) centres + --sigma noise, --clusters of\n"
    "          them; codes: uniform codes with N(0,1) codebooks, no base vectors)\n"
    "search:   --m --nq --k --rerank R\n"
    "training: --train --iters\n"
    "measure:  --reps --eval-queries (0 = skip recall) --cpu-queries (0 = skip CPU)\n"
    "gpu:      --variants all|v0,v1,...,v8[,v9]  --threads T  --blocks-per-query B  --queries-per-block Q  --ilp 1|2|4\n"
    "output:   --csv out.csv  --label name";

Settings parse_settings(int argc, char** argv) {
    Settings s;
    const std::vector<Flag> flags = flag_table(s);
    for (int i = 1; i < argc; ++i) {
        const std::string name = argv[i];
        if (name == "-h" || name == "--help") {
            std::puts(kUsage);
            std::exit(0);
        }
        const auto f = std::find_if(flags.begin(), flags.end(), [&](const Flag& x) { return name == x.name; });
        if (f == flags.end()) throw std::runtime_error("unknown option " + name + " (try --help)");
        check(i + 1 < argc, "missing value for " + name);
        f->set(argv[++i]);
    }
    check(s.k >= 1 && s.k <= 128, "--k must be in [1, 128]");
    return s;
}

// "all" selects the reference's registry (v0 .. v8); otherwise comma-separated name prefixes ("v2,v8" or full names).
bool selected(const std::string& list, gpu::ScanVariant v) {
    const std::string name = gpu::variant_name(v);
    if (list == "all") return v != gpu::ScanVariant::FusedWarpF16;
    std::istringstream items(list);
    for (std::string item; std::getline(items, item, ',');)
        if (!item.empty() && name.rfind(item, 0) == 0) return true;
    return false;
}

bool needs_m16(gpu::ScanVariant v) {
    using V = gpu::ScanVariant;
    return v == V::SharedLutVec || v == V::FusedVec || v == V::FusedVecMQ || v == V::FusedWarp || v == V::FusedWarpF16;
}

// ------------------------------------------------------------------------------------------------ dataset, index

struct Dataset {
    std::vector<float> base, queries;
    std::vector<uint8_t> codes;     // filled for --data codes only
    std::vector<float> codebook;    // idem
    std::string source;
};

std::vector<float> read_rows(const std::string& path, std::size_t& n, std::size_t& d, std::size_t max_n) {
    const bool bytes = path.size() >= 6 && path.compare(path.size() - 6, 6, ".bvecs") == 0;
    return bytes ? read_bvecs(path, n, d, max_n) : read_fvecs(path, n, d, max_n);
}

Dataset load_dataset(Settings& s) {
    Dataset ds;
    if (!s.base.empty()) {
        check(!s.query.empty(), "--base requires --query");
        ds.base = read_rows(s.base, s.n, s.d, s.n);
        std::size_t qd = 0;
        ds.queries = read_rows(s.query, s.nq, qd, s.nq);
        check(qd == s.d, "query and base dimensions differ");
        ds.source = "files";
        return ds;
    }
    const std::size_t query_rows = std::size_t{1} << 40;  // queries: a row range of the source disjoint from the base
    ds.queries.resize(s.nq * s.d);
    if (s.data == "codes") {
        check(s.d % s.m == 0, "d must be a multiple of m");
        ds.codes.resize(s.n * s.m);
        uniform_codes(0, s.n, s.m, s.seed, ds.codes.data());
        ds.codebook.resize(s.m * kSubCentroids * (s.d / s.m));
        normal_values(s.seed, 30, 0, ds.codebook.size(), ds.codebook.data());
        normal_values(s.seed, 31, 0, ds.queries.size(), ds.queries.data());
        s.eval_queries = 0;  // no base vectors, so no exact ground truth
        s.cpu_queries = std::min(s.cpu_queries, s.nq);
        ds.source = "codes";
        return ds;
    }
    ds.base.resize(s.n * s.d);
    if (s.data == "latent") {
        const SyntheticSource src(s.d, s.clusters, s.seed, s.latent_dim);
        src.fill(0, s.n, ds.base.data());
        src.fill(query_rows, s.nq, ds.queries.data());
    } else {
        check(s.data == "mixture", "--data must be latent, mixture or codes");
        const GaussianMixture src(s.d, s.clusters, static_cast<float>(s.sigma), s.seed);
        src.fill(0, s.n, ds.base.data());
        src.fill(query_rows, s.nq, ds.queries.data());
    }
    ds.source = s.data;
    return ds;
}

// The codebook and the codes the searches run on.
ProductQuantizer build_index(const Settings& s, Dataset& ds) {
    ProductQuantizer pq(s.d, s.m);
    if (!ds.codebook.empty()) {
        pq.set_centroids(ds.codebook);
        return pq;
    }
    pq.train(ds.base.data(), std::min(s.train, s.n), s.iters, s.seed);
    ds.codes.resize(s.n * s.m);
    pq.encode(ds.base.data(), s.n, ds.codes.data());
    return pq;
}

// ------------------------------------------------------------------------------------------------ scoring

// Recall@k of result rows for the first `queries` queries. With --rerank R the rows hold R candidates, which are
// re-ranked exactly (on the GPU; the same results as the reference's CPU rerank_exact) before scoring.
class Scorer {
public:
    Scorer(const Settings& s, const Dataset& ds) : k_(s.k), rerank_(s.rerank), queries_(s.eval_queries), ds_(ds) {
        if (queries_ == 0) return;
        if (!s.gt.empty()) {
            std::size_t rows = 0;
            truth_ = read_ivecs(s.gt, rows, stride_, s.nq);
            check(rows >= queries_ && stride_ >= k_, "ground truth too small");
        } else {
            const Timer clock;
            std::vector<Neighbor> exact(queries_ * k_);
            exact_knn(ds.base.data(), s.n, ds.queries.data(), queries_, s.d, k_, exact.data());
            truth_.resize(exact.size());
            std::transform(exact.begin(), exact.end(), truth_.begin(), [](const Neighbor& x) { return x.id; });
            stride_ = k_;
            std::printf("exact ground truth (%zu queries): %.1f s\n", queries_, clock.ms() / 1e3);
        }
        if (rerank_) reranker_ = std::make_unique<gpu::Reranker>(ds.base.data(), s.n, s.d);
    }

    std::size_t result_width() const { return rerank_ ? std::max(k_, rerank_) : k_; }
    gpu::Reranker* reranker() const { return reranker_.get(); }

    // rows: at least `queries_` rows of result_width() neighbours. -1 when recall is not measured.
    double recall(const std::vector<Neighbor>& rows) const {
        if (queries_ == 0) return -1.0;
        const std::size_t width = result_width();
        if (!rerank_) return recall_at_k(rows.data(), width, truth_.data(), stride_, queries_, k_);
        std::vector<Neighbor> best(queries_ * k_);
        reranker_->rerank(ds_.queries.data(), queries_, rows.data(), width, k_, best.data());
        return recall_at_k(best.data(), k_, truth_.data(), stride_, queries_, k_);
    }

    std::size_t queries() const { return queries_; }

private:
    std::size_t k_, rerank_, queries_, stride_ = 0;
    const Dataset& ds_;
    std::vector<int32_t> truth_;
    std::unique_ptr<gpu::Reranker> reranker_;
};

// ------------------------------------------------------------------------------------------------ rows

struct Row {
    std::string variant;
    gpu::PQSearcher::LaunchShape shape;
    gpu::Timings t;  // per-stage medians (the CPU row: total in transfer-free scan_ms)
    double total_ms = 0, qps = 0, code_gbs = 0, recall = -1;
};

double median_of(std::vector<double> v) {
    if (v.empty()) return 0.0;
    std::nth_element(v.begin(), v.begin() + v.size() / 2, v.end());
    return v[v.size() / 2];
}

int host_cores() {
    const long online = sysconf(_SC_NPROCESSORS_ONLN);
    return online > 0 ? static_cast<int>(online) : 1;
}

int omp_threads() {
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}

// The CPU search path on the first cpu_queries queries, timed as one call (the reference's cpu_reference row).
Row cpu_row(const Settings& s, const ProductQuantizer& pq, const Dataset& ds, const Scorer& scorer) {
    const std::size_t q = std::min(s.cpu_queries, s.nq), width = scorer.result_width();
    std::vector<Neighbor> res(q * width);
    const Timer clock;
    adc_search(pq, ds.codes.data(), s.n, ds.queries.data(), q, width, res.data());
    Row r;
    r.variant = "cpu_reference";
    r.total_ms = clock.ms();
    r.shape.threads = omp_threads();  // the T column of the CPU row: OpenMP threads
    r.qps = q / (r.total_ms / 1e3);
    r.code_gbs = static_cast<double>(s.n) * s.m * q / (r.total_ms / 1e3) / 1e9;
    if (q >= scorer.queries()) r.recall = scorer.recall(res);
    std::printf("cpu_reference: %zu queries on %d OpenMP threads (%d host cores online): %.1f ms\n", q,
                omp_threads(), host_cores(), r.total_ms);
    return r;
}

// One GPU variant: an untimed call (it also builds the variant's code layout), then reps timed calls.
Row gpu_row(const Settings& s, gpu::PQSearcher& searcher, gpu::ScanVariant v, const Dataset& ds,
            const Scorer& scorer) {
    const std::size_t width = scorer.result_width();
    std::vector<Neighbor> res(s.nq * width);
    searcher.search(ds.queries.data(), s.nq, width, v, res.data());
    std::vector<double> transfer, lut, scan, select, total;
    for (std::size_t rep = 0; rep < s.reps; ++rep) {
        const gpu::Timings t = searcher.search(ds.queries.data(), s.nq, width, v, res.data());
        transfer.push_back(t.transfer_ms);
        lut.push_back(t.lut_ms);
        scan.push_back(t.scan_ms);
        select.push_back(t.select_ms);
        total.push_back(t.total_ms());
    }
    Row r;
    r.variant = gpu::variant_name(v);
    r.shape = searcher.last_launch();
    r.t.transfer_ms = median_of(transfer);
    r.t.lut_ms = median_of(lut);
    r.t.scan_ms = median_of(scan);
    r.t.select_ms = median_of(select);
    r.total_ms = median_of(total);
    r.qps = s.nq / (r.total_ms / 1e3);
    r.code_gbs = static_cast<double>(s.n) * s.m * s.nq / (r.t.scan_ms / 1e3) / 1e9;
    if (gpu::Reranker* rr = scorer.reranker()) {  // the re-rank of the whole batch, timed apart from the search
        std::vector<Neighbor> best(s.nq * s.k);
        std::vector<double> ms;
        for (std::size_t rep = 0; rep <= s.reps; ++rep) {
            const gpu::Timings t = rr->rerank(ds.queries.data(), s.nq, res.data(), width, s.k, best.data());
            if (rep > 0) ms.push_back(t.scan_ms);
        }
        std::printf("%s: exact GPU re-rank of %zu x %zu candidates to k=%zu: %.3f ms kernel\n", r.variant.c_str(),
                    s.nq, width, s.k, median_of(ms));
    }
    res.resize(std::max<std::size_t>(scorer.queries(), 1) * width);
    r.recall = scorer.recall(res);
    return r;
}

// ------------------------------------------------------------------------------------------------ report

void print_table(const std::vector<Row>& rows) {
    std::printf("\n%-18s %5s %5s %5s %2s %3s %5s %8s %8s %8s %8s %9s %10s %9s %7s\n", "variant", "T", "bx", "gy", "Q",
                "ILP", "waves", "lut ms", "scan ms", "sel ms", "xfer ms", "total ms", "QPS", "code GB/s", "recall");
    for (const Row& r : rows)
        std::printf("%-18s %5d %5d %5d %2d %3d %5.2f %8.3f %8.3f %8.3f %8.3f %9.3f %10.0f %9.1f %7.3f\n",
                    r.variant.c_str(), r.shape.threads, r.shape.blocks_x, r.shape.grid_y, r.shape.queries_per_block,
                    r.shape.vectors_per_step, r.shape.waves, r.t.lut_ms, r.t.scan_ms, r.t.select_ms, r.t.transfer_ms,
                    r.total_ms, r.qps, r.code_gbs, r.recall);
    std::puts("code GB/s = logical PQ code bytes per query x queries / scan time (CPU row: whole search); it counts "
              "L2 and MALL hits. CPU row: T = OpenMP threads.");
}

void append_csv(const Settings& s, const std::vector<Row>& rows) {
    const bool fresh = !std::ifstream(s.csv).good();
    std::ofstream out(s.csv, std::ios::app);
    if (fresh)
        out << "label,variant,n,d,m,nq,k,rerank,threads,blocks_x,grid_y,qpb,ilp,blocks_per_sm,waves,lut_ms,scan_ms,"
               "select_ms,transfer_ms,total_ms,qps,code_gbs,recall\n";
    for (const Row& r : rows) {
        const auto& sh = r.shape;
        out << s.label << ',' << r.variant << ',' << s.n << ',' << s.d << ',' << s.m << ',' << s.nq << ',' << s.k
            << ',' << s.rerank << ',' << sh.threads << ',' << sh.blocks_x << ',' << sh.grid_y << ','
            << sh.queries_per_block << ',' << sh.vectors_per_step << ',' << sh.blocks_per_sm << ',' << sh.waves << ','
            << r.t.lut_ms << ',' << r.t.scan_ms << ',' << r.t.select_ms << ',' << r.t.transfer_ms << ','
            << r.total_ms << ',' << r.qps << ',' << r.code_gbs << ',' << r.recall << '\n';
    }
    std::printf("appended %zu rows to %s\n", rows.size(), s.csv.c_str());
}

int run(int argc, char** argv) {
    Settings s = parse_settings(argc, argv);
    const Timer data_clock;
    Dataset ds = load_dataset(s);
    s.eval_queries = std::min(s.eval_queries, s.nq);
    s.cpu_queries = std::min(s.cpu_queries, s.nq);
    std::printf("data: n=%zu d=%zu nq=%zu (%s, %.1f s) | PQ m=%zu (%zu B/vector, %.0fx compression) | k=%zu\n", s.n,
                s.d, s.nq, ds.source.c_str(), data_clock.ms() / 1e3, s.m, s.m, 4.0 * s.d / s.m, s.k);

    const Timer index_clock;
    const ProductQuantizer pq = build_index(s, ds);
    std::printf("PQ train+encode: %.1f s\n", index_clock.ms() / 1e3);
    check(!s.rerank || !ds.base.empty(), "--rerank needs base vectors (not available with --data codes)");
    const Scorer scorer(s, ds);

    std::vector<Row> rows;
    if (s.cpu_queries > 0) rows.push_back(cpu_row(s, pq, ds, scorer));

    const gpu::DeviceInfo info = gpu::device_info();
    std::printf("GPU: %s, %d CUs, %.0f GB/s theoretical HBM peak, %zu B LDS per block\n", info.name.c_str(),
                info.sm_count, info.peak_bandwidth_gbs, info.max_smem_per_block);
    gpu::PQSearcher searcher(pq, ds.codes.data(), s.n);
    gpu::Tuning tuning;
    tuning.scan_threads = static_cast<int>(s.threads);
    tuning.blocks_per_query = static_cast<int>(s.blocks_per_query);
    tuning.queries_per_block = static_cast<int>(s.queries_per_block);
    tuning.vectors_per_step = static_cast<int>(s.ilp);
    searcher.set_tuning(tuning);
    for (int i = 0; i <= static_cast<int>(gpu::ScanVariant::FusedWarpF16); ++i) {
        const auto v = static_cast<gpu::ScanVariant>(i);
        if (!selected(s.variants, v) || (needs_m16(v) && s.m % 16 != 0)) continue;
        try {
            rows.push_back(gpu_row(s, searcher, v, ds, scorer));
        } catch (const std::logic_error& e) {  // a variant this build does not launch (v4): no row, the run goes on
            std::printf("%s: no row (%s)\n", gpu::variant_name(v), e.what());
        }
    }

    print_table(rows);
    append_csv(s, rows);
    return 0;
}

}  // namespace

int main(int argc, char** argv) {
    try {
        return run(argc, argv);
    } catch (const std::exception& e) {
        std::fprintf(stderr, "error: %s\n", e.what());
        return 1;
    }
}
