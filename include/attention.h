/*
 * attention.h - the reference's single-query attention API, served by the
 * MI355X library.
 *
 * Same names, arguments and return values as the reference header
 * (reference attention/src/attention.h:27-208).  Inputs are host pointers,
 * row-major fp32: Q [1 x d], K and V [T x d]; results come back by value.
 * Every variant runs the split-KV online-softmax kernel of libsa_amd on the
 * current HIP device and returns after the result is on the host; the
 * thread-count, NUMA and MPI arguments of the reference do not change the
 * GPU computation.
 *
 * Differences from the reference, all deliberate:
 *   - d must be 8, 16, 32, 64, 128 or 256 (the kernels' head sizes); other
 *     values throw std::invalid_argument instead of computing.
 *   - block_size must be positive (the reference divides by it).
 *   - T <= 0 returns zeros for every variant (streaming_attention_omp of the
 *     reference returns NaN for T = 0).
 *   - The _mpi variants run as the single rank 0: T_local must equal
 *     T_global, and comm is not used.
 */
#ifndef SA_AMD_ATTENTION_H
#define SA_AMD_ATTENTION_H

#include <vector>

#if !defined(MPI_COMM_WORLD) && !defined(OMPI_MPI_H) && !defined(MPICH_NAME) && !defined(MPI_VERSION) && \
    !defined(MPI_Comm)
typedef void* MPI_Comm;
#endif

/* O = softmax(Q K^T) V, three-pass form (reference attention/src/naive_serial.cpp:18-72). */
std::vector<float> naive_attention_serial(const float* Q, const float* K, const float* V, int T, int d);

/* reference attention/src/naive_omp.cpp:24-90 */
std::vector<float> naive_attention_omp(const float* Q, const float* K, const float* V, int T, int d,
                                       int num_threads = 0);

/* reference attention/src/naive_mpi.cpp (single rank here) */
std::vector<float> naive_attention_mpi(const float* Q_local, const float* K_local, const float* V_local,
                                       int T_local, int T_global, int d, int num_omp_threads, MPI_Comm comm);

std::vector<float> naive_attention_mpi_simple(const float* Q_local, const float* K_local,
                                              const float* V_local, int T_local, int T_global, int d,
                                              MPI_Comm comm);

/* Online-softmax block attention (reference attention/src/streaming_serial.cpp:20-71). */
std::vector<float> streaming_attention_serial(const float* Q, const float* K, const float* V, int T, int d,
                                              int block_size);

/* Relative L2 error ||a-b|| / ||b|| (absolute when ||b|| < 1e-10) and max
 * absolute error (reference attention/src/naive_serial.cpp:75-98). */
float compute_l2_error(const float* a, const float* b, int size);
float compute_max_error(const float* a, const float* b, int size);

/* reference attention/src/streaming_omp.cpp:99-154 */
std::vector<float> streaming_attention_omp(const float* Q, const float* K, const float* V, int T, int d,
                                           int block_size, int num_threads = 0);

/* reference attention/src/streaming_omp.cpp:162-174 */
std::vector<float> streaming_attention_omp_numa(const float* Q, const float* K, const float* V, int T,
                                                int d, int block_size, int num_threads = 0);

/* reference attention/src/streaming_mpi.cpp:252-309 (single rank here) */
std::vector<float> streaming_attention_mpi_simple(const float* Q_local, const float* K_local,
                                                  const float* V_local, int T_local, int T_global, int d,
                                                  int block_size, MPI_Comm comm);

#endif /* SA_AMD_ATTENTION_H */
