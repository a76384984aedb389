// lxm_runner: replay a packed decode (written by linuxformer_amd.mega.Mega.dump) through the C ABI
// of liblxm.so, without Python: the binding a foreign host (C, Go via cgo, ...) would use, and the
// process rocprofv3 profiles.
//
//   lxm_runner <dump dir> <launches> [tokens per launch, at most the dumped count]
//   lxm_runner --copy <MiB>     (one plain device copy kernel of that size: the calibration run
//                                for the HBM byte counters FETCH_SIZE and WRITE_SIZE)
//
// The dump's manifest lists each lxm_params pointer field with the file holding its device
// buffer ("buf"), a zeroed buffer size ("zero"), or a list of files whose device copies form a
// pointer array ("ptrs", the per-layer states), or a pointer into another buffer ("sub"). Every launch continues the stream from the last
// prediction of the one before. Prints one JSON line: tokens, per-launch kernel milliseconds
// (hipEvent), tok/s, the last prediction.
#include <dlfcn.h>
#include <hip/hip_runtime.h>

#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <fstream>
#include <map>
#include <sstream>
#include <string>
#include <vector>

#include "../../include/lxm.h"

#define CK(x)                                                                    \
  do {                                                                           \
    hipError_t e_ = (x);                                                         \
    if (e_ != hipSuccess) {                                                      \
      fprintf(stderr, "%s:%d %s\n", __FILE__, __LINE__, hipGetErrorString(e_)); \
      exit(1);                                                                   \
    }                                                                            \
  } while (0)

static std::vector<char> slurp(const std::string& path) {
  std::ifstream f(path, std::ios::binary);
  if (!f) {
    fprintf(stderr, "cannot read %s\n", path.c_str());
    exit(1);
  }
  return std::vector<char>((std::istreambuf_iterator<char>(f)), std::istreambuf_iterator<char>());
}

static std::vector<void*> g_allocs;  // every device buffer the runner made, freed at the end

static void* dev_alloc(size_t n) {
  void* d = nullptr;
  CK(hipMalloc(&d, n));
  g_allocs.push_back(d);
  return d;
}

static void* upload(const std::string& path, size_t* n = nullptr) {
  std::vector<char> b = slurp(path);
  void* d = dev_alloc(b.size() + 256);
  CK(hipMemcpy(d, b.data(), b.size(), hipMemcpyHostToDevice));
  if (n) *n = b.size();
  return d;
}

// a grid-stride copy of n 16-byte words
__global__ void copy16(const uint4* __restrict__ src, uint4* __restrict__ dst, size_t n) {
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x)
    dst[i] = src[i];
}

static int copy_run(size_t mib) {
  const size_t bytes = mib << 20, n = bytes / 16;
  void *a = nullptr, *b = nullptr;
  CK(hipMalloc(&a, bytes));
  CK(hipMalloc(&b, bytes));
  CK(hipMemset(a, 1, bytes));
  CK(hipDeviceSynchronize());
  hipLaunchKernelGGL(copy16, dim3(4096), dim3(256), 0, 0, (const uint4*)a, (uint4*)b, n);
  CK(hipGetLastError());
  CK(hipDeviceSynchronize());
  printf("{\"copy_bytes_read\": %zu, \"copy_bytes_written\": %zu}\n", bytes, bytes);
  fflush(stdout);
  CK(hipFree(a));
  CK(hipFree(b));
  return 0;
}

int main(int argc, char** argv) {
  if (argc == 3 && std::string(argv[1]) == "--copy") return copy_run((size_t)atol(argv[2]));
  if (argc < 3) {
    fprintf(stderr, "usage: %s <dump dir> <launches> [tokens]\n", argv[0]);
    return 2;
  }
  const std::string dir = argv[1];
  const int launches = atoi(argv[2]);
  std::string libpath = std::string(getenv("LXM_LIB") ? getenv("LXM_LIB") : "");
  if (libpath.empty()) {
    std::ifstream lf(dir + "/lib.txt");
    std::getline(lf, libpath);
  }
  void* h = dlopen(libpath.c_str(), RTLD_NOW);
  if (!h) {
    fprintf(stderr, "dlopen %s: %s\n", libpath.c_str(), dlerror());
    return 1;
  }
  auto run = (int (*)(const lxm_params*, const lxm_params*, int, int, void*))dlsym(h, "lxm_run");
  auto last = (int (*)(void))dlsym(h, "lxm_last_error");
  if (!run || !last) return 1;

  std::vector<char> pb = slurp(dir + "/params.bin");
  if (pb.size() != sizeof(lxm_params)) {
    fprintf(stderr, "params.bin: %zu bytes, lxm_params is %zu\n", pb.size(), sizeof(lxm_params));
    return 1;
  }
  lxm_params p;
  memcpy(&p, pb.data(), sizeof p);
  std::map<std::string, void**> field = {
      {"layers", (void**)&p.layers},     {"blob", (void**)&p.blob},
      {"gates", (void**)&p.gates},
      {"rec", (void**)&p.rec},           {"conv", (void**)&p.conv},
      {"emb_ptr", (void**)&p.emb_ptr},   {"emb_ent", (void**)&p.emb_ent},
      {"w1_final", (void**)&p.w1_final}, {"head_rows", (void**)&p.head_rows},
      {"head_ptr", (void**)&p.head_ptr}, {"head_ent", (void**)&p.head_ent},
      {"forced", (void**)&p.forced},     {"preds", (void**)&p.preds},
      {"inputs", (void**)&p.inputs},     {"trace", (void**)&p.trace},
      {"ring", (void**)&p.ring},         {"hn", (void**)&p.hn},
      {"rring", (void**)&p.rring},
      {"sync", (void**)&p.sync},         {"keys", (void**)&p.keys},
      {"err", (void**)&p.err},           {"prof", (void**)&p.prof},
      {"mb_task", (void**)&p.mb_task},   {"mb_e", (void**)&p.mb_e},
      {"mb_qk", (void**)&p.mb_qk},       {"ybuf", (void**)&p.ybuf},
      {"xo", (void**)&p.xo},             {"head_dcol", (void**)&p.head_dcol},
      {"head_dtab", (void**)&p.head_dtab}, {"head_code", (void**)&p.head_code}};
  for (auto& kv : field) *kv.second = nullptr;
  int n_blocks = 0, lds = 0;
  std::vector<std::string> manifest;
  {
    std::ifstream mf(dir + "/manifest.txt");
    for (std::string l; std::getline(mf, l);) manifest.push_back(l);
  }
  std::map<std::string, size_t> zero_bytes;  // the size of each zeroed buffer, by field
  for (const std::string& line : manifest) {
    std::istringstream ss(line);
    std::string kind, name;
    size_t n = 0;
    if ((ss >> kind >> name) && kind == "zero" && (ss >> n)) zero_bytes[name] = n;
  }
  {
    // the launch writes n_tokens predictions (and inputs / a trace when the dump has them):
    // refuse a count its buffers cannot hold, before anything touches the GPU
    const long n = argc > 3 ? atol(argv[3]) : (long)p.n_tokens;
    const size_t per_trace = (size_t)p.n_layers * p.hidden * 4;
    auto holds = [&](const char* f, size_t need) {
      return zero_bytes.count(f) && need <= zero_bytes.at(f);
    };
    const bool fits = n >= 1 && holds("preds", (size_t)n * 4) &&
                      (!zero_bytes.count("inputs") || holds("inputs", (size_t)n * 4)) &&
                      (!zero_bytes.count("trace") || holds("trace", (size_t)n * per_trace));
    if (!fits) {
      fprintf(stderr, "tokens %ld: the dump's buffers hold %zu predictions (dump again with more)\n",
              n, zero_bytes.count("preds") ? zero_bytes.at("preds") / 4 : (size_t)0);
      return 2;
    }
    p.n_tokens = (int)n;
  }
  for (const std::string& line : manifest) {
    std::istringstream ss(line);
    std::string kind, name;
    ss >> kind >> name;
    if (kind == "launch") {
      ss >> n_blocks >> lds;
    } else if (kind == "buf") {
      std::string file;
      ss >> file;
      *field.at(name) = upload(dir + "/" + file);
    } else if (kind == "zero") {
      size_t n;
      ss >> n;
      void* d = dev_alloc(n);
      CK(hipMemset(d, 0, n));
      *field.at(name) = d;
    } else if (kind == "sub") {  // a pointer into another buffer: sub <field> <base field> <offset>
      std::string base;
      size_t off;
      ss >> base >> off;
      *field.at(name) = (char*)*field.at(base) + off;
    } else if (kind == "ptrs") {
      int n;
      ss >> n;
      std::vector<void*> ptrs(n);
      for (int i = 0; i < n; i++) {
        std::string file;
        ss >> file;
        ptrs[i] = upload(dir + "/" + file);
      }
      void* d = dev_alloc(sizeof(void*) * n);
      CK(hipMemcpy(d, ptrs.data(), sizeof(void*) * n, hipMemcpyHostToDevice));
      *field.at(name) = d;
    }
  }
  int* forced_d = (int*)p.forced;
  int* preds_d = p.preds;
  lxm_params* pd = (lxm_params*)dev_alloc(sizeof p);
  hipStream_t st;
  CK(hipStreamCreate(&st));
  hipEvent_t e0, e1;
  CK(hipEventCreate(&e0));
  CK(hipEventCreate(&e1));
  std::vector<float> ms;
  int tok = 0;
  CK(hipMemcpy(&tok, forced_d, 4, hipMemcpyDeviceToHost));
  for (int k = 0; k < launches; k++) {
    // sync words, keys, the value heads' stamped outputs and the error flag start at zero; the
    // stream continues from `tok`
    CK(hipMemsetAsync(p.sync, 0, LXM_NSYNC * 4, st));
    CK(hipMemsetAsync(p.keys, 0, 16, st));
    CK(hipMemsetAsync(p.ybuf, 0, (size_t)p.nv * p.vd * 8, st));
    CK(hipMemsetAsync(p.err, 0, 4, st));
    CK(hipMemcpyAsync(forced_d, &tok, 4, hipMemcpyHostToDevice, st));
    p.n_forced = 1;
    CK(hipMemcpyAsync(pd, &p, sizeof p, hipMemcpyHostToDevice, st));
    CK(hipEventRecord(e0, st));
    int rc = run(&p, pd, n_blocks, lds, st);
    if (rc) {
      fprintf(stderr, "lxm_run: hipError %d\n", rc);
      return 1;
    }
    CK(hipEventRecord(e1, st));
    CK(hipStreamSynchronize(st));
    float t = 0;
    CK(hipEventElapsedTime(&t, e0, e1));
    ms.push_back(t);
    int err = 0;
    CK(hipMemcpy(&err, p.err, 4, hipMemcpyDeviceToHost));
    if (err || last()) {
      fprintf(stderr, "decode failed: err %d\n", err);
      return 1;
    }
    CK(hipMemcpy(&tok, preds_d + p.n_tokens - 1, 4, hipMemcpyDeviceToHost));
    fprintf(stderr, "[lxm_runner] launch %d/%d: %d tokens in %.3f ms\n", k + 1, launches,
            p.n_tokens, t);
  }
  double tot = 0;
  for (float t : ms) tot += t;
  printf("{\"tokens_per_launch\": %d, \"launches\": %d, \"kernel_ms\": [", p.n_tokens, launches);
  for (size_t i = 0; i < ms.size(); i++) printf("%s%.3f", i ? ", " : "", ms[i]);
  printf("], \"tok_per_s\": %.1f, \"last_pred\": %d}\n", p.n_tokens * launches / (tot * 1e-3), tok);
  fflush(stdout);
  // teardown in dependency order, while the runtime is up: the stream's work, the events and the
  // stream, every device buffer, then the library (its code object unregisters before exit)
  CK(hipStreamSynchronize(st));
  CK(hipEventDestroy(e0));
  CK(hipEventDestroy(e1));
  CK(hipStreamDestroy(st));
  for (void* d : g_allocs) CK(hipFree(d));
  g_allocs.clear();
  CK(hipDeviceSynchronize());
  dlclose(h);
  return 0;
}
