// cpu_baselines.cpp -- labelled C++ stand-ins for the reference benchmark's
// CPU baselines (metal-forge-compute/forge-sort/benches/sort_benchmark.rs:176-177:
// Rust slice::sort_unstable and rayon par_sort_unstable), used only by the
// cpu_baseline leg of bench.py.  Rust is not available on this machine, so
//   std::sort                 stands in for sort_unstable (1 thread)
//   __gnu_parallel::sort      stands in for par_sort_unstable (OpenMP threads)
// Both are comparison sorts of u32 keys, like the reference's baselines.
#include <parallel/algorithm>
#include <omp.h>
#include <stdint.h>
#include <algorithm>

extern "C" {

void cb_std_sort_u32(uint32_t* keys, uint64_t n) { std::sort(keys, keys + n); }

void cb_parallel_sort_u32(uint32_t* keys, uint64_t n, int threads) {
    omp_set_num_threads(threads);
    __gnu_parallel::sort(keys, keys + n);
}

int cb_max_threads(void) { return omp_get_max_threads(); }

}
