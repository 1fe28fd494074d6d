// neptune_abi_caller.cpp — a native C++ host driving libneptune_hip.so
// through include/neptune_hip.h only, the way a C++ runtime (the
// reference's own plugin host: dlopen + extern "C" entry points,
// lib/HTile/HTileDialect.cpp:27-37) would. It owns every device buffer
// (hipMalloc / hipMemcpy), calls the C-ABI, and checks the results itself.
//
//   neptune_abi_caller validate      status codes of the host-side checks;
//                                     the no-device path where no GPU exists
//   neptune_abi_caller attn DIR      neptune_attn_fwd on DIR's fixture
//   neptune_abi_caller decode DIR    neptune_decode_splitk (caller workspace)
//                                     and neptune_decode_splitk_noalloc on it
//
// DIR holds meta.txt ("key value" lines) and raw little-endian arrays:
// q.bin k.bin v.bin (bf16 bits), o.bin and lse.bin (float32, expected).
// Exit status 0 = every check passed; the last line says what was checked.
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <fstream>
#include <map>
#include <sstream>
#include <string>
#include <vector>

#include "neptune_hip.h"

namespace {

int g_failures = 0;

void expect(bool ok, const char *what) {
  if (!ok) {
    std::fprintf(stderr, "FAIL: %s (last error: %s)\n", what, neptune_last_error());
    ++g_failures;
  }
}

std::map<std::string, double> read_meta(const std::string &dir) {
  std::map<std::string, double> m;
  std::ifstream f(dir + "/meta.txt");
  std::string key;
  double val;
  while (f >> key >> val) m[key] = val;
  return m;
}

template <class T>
std::vector<T> read_array(const std::string &path) {
  std::ifstream f(path, std::ios::binary | std::ios::ate);
  if (!f) {
    std::fprintf(stderr, "cannot open %s\n", path.c_str());
    std::exit(2);
  }
  const std::streamsize n = f.tellg();
  std::vector<T> v(static_cast<size_t>(n) / sizeof(T));
  f.seekg(0);
  f.read(reinterpret_cast<char *>(v.data()), n);
  return v;
}

float bf16_to_f32(uint16_t b) {
  const uint32_t u = static_cast<uint32_t>(b) << 16;
  float f;
  std::memcpy(&f, &u, 4);
  return f;
}

bool hip_ok(hipError_t e, const char *what) {
  if (e != hipSuccess) {
    std::fprintf(stderr, "FAIL: %s: %s\n", what, hipGetErrorString(e));
    ++g_failures;
    return false;
  }
  return true;
}

// A device copy of a host array, freed with the object.
struct DeviceBuffer {
  void *ptr = nullptr;
  size_t bytes = 0;
  explicit DeviceBuffer(size_t n) : bytes(n) { hip_ok(hipMalloc(&ptr, n ? n : 1), "hipMalloc"); }
  template <class T>
  explicit DeviceBuffer(const std::vector<T> &host) : DeviceBuffer(host.size() * sizeof(T)) {
    hip_ok(hipMemcpy(ptr, host.data(), bytes, hipMemcpyHostToDevice), "copy to device");
  }
  template <class T>
  std::vector<T> to_host() const {
    std::vector<T> v(bytes / sizeof(T));
    hip_ok(hipMemcpy(v.data(), ptr, bytes, hipMemcpyDeviceToHost), "copy to host");
    return v;
  }
  ~DeviceBuffer() {
    if (ptr) (void)hipFree(ptr);
  }
  DeviceBuffer(const DeviceBuffer &) = delete;
  DeviceBuffer &operator=(const DeviceBuffer &) = delete;
};

// max |got - want| over bf16 outputs against float32 expectations
double max_err_bf16(const std::vector<uint16_t> &got, const std::vector<float> &want) {
  double e = 0.0;
  for (size_t i = 0; i < want.size(); ++i)
    e = std::fmax(e, std::fabs((double)bf16_to_f32(got[i]) - (double)want[i]));
  return e;
}

double max_err_f32(const std::vector<float> &got, const std::vector<float> &want) {
  double e = 0.0;
  for (size_t i = 0; i < want.size(); ++i) e = std::fmax(e, std::fabs((double)got[i] - want[i]));
  return e;
}

neptune_attn_desc attn_desc(int64_t b, int64_t hq, int64_t hk, int64_t sq, int64_t sk,
                            int64_t d) {
  neptune_attn_desc a;
  std::memset(&a, 0, sizeof a);
  a.batch = b; a.heads_q = hq; a.heads_kv = hk; a.seq_q = sq; a.seq_kv = sk; a.head_dim = d;
  a.dtype = NEPTUNE_DTYPE_BF16;
  return a;
}

neptune_decode_desc decode_desc(int64_t b, int64_t hq, int64_t hk, int64_t l, int64_t splits) {
  neptune_decode_desc d;
  std::memset(&d, 0, sizeof d);
  d.batch = b; d.heads_q = hq; d.heads_kv = hk; d.seq_kv = l; d.head_dim = 128;
  d.num_splits = splits;
  d.q_dtype = NEPTUNE_DTYPE_BF16;
  d.kv_dtype = NEPTUNE_DTYPE_BF16;
  return d;
}

int run_validate() {
  neptune_backend_info info;
  expect(neptune_hip_get_backend_info(&info) == NEPTUNE_OK, "backend info");
  expect(info.abi_version == NEPTUNE_HIP_ABI_VERSION, "abi version");
  expect(std::strcmp(info.name, "NeptuneHTileHIP") == 0, "backend name");
  expect(std::strcmp(info.gcn_arch, "gfx950") == 0, "gcn arch");
  expect(neptune_hip_get_backend_info(nullptr) == NEPTUNE_ERR_INVALID_ARGUMENT, "null info");

  // placeholder device addresses: every call below fails validation first
  void *fake = reinterpret_cast<void *>(uintptr_t(0x10000));
  neptune_attn_desc a = attn_desc(1, 4, 2, 256, 256, 128);
  expect(neptune_attn_fwd(nullptr, fake, fake, fake, fake, nullptr, nullptr) ==
             NEPTUNE_ERR_INVALID_ARGUMENT, "attn: null desc");
  neptune_attn_desc bad = a;
  bad.heads_kv = 3;
  expect(neptune_attn_fwd(&bad, fake, fake, fake, fake, nullptr, nullptr) ==
             NEPTUNE_ERR_INVALID_ARGUMENT, "attn: heads_q % heads_kv");
  bad = a;
  bad.head_dim = 96;
  expect(neptune_attn_fwd(&bad, fake, fake, fake, fake, nullptr, nullptr) ==
             NEPTUNE_ERR_UNSUPPORTED, "attn: head_dim 96");
  expect(std::strlen(neptune_last_error()) > 0, "attn: error text");
  bad = a;
  bad.v_stride[0] = 1 << 30; bad.v_stride[1] = 1 << 28; bad.v_stride[2] = 34100000 / 8 * 8;
  bad.q_stride[0] = bad.k_stride[0] = bad.o_stride[0] = 1 << 30;
  bad.q_stride[1] = bad.k_stride[1] = bad.o_stride[1] = 1 << 28;
  bad.q_stride[2] = bad.k_stride[2] = bad.o_stride[2] = 128;
  expect(neptune_attn_fwd(&bad, fake, fake, fake, fake, nullptr, nullptr) ==
             NEPTUNE_ERR_UNSUPPORTED, "attn: V tile past 32-bit offsets");

  neptune_decode_desc d = decode_desc(2, 8, 2, 1000, 3);
  size_t ws = 0;
  expect(neptune_decode_workspace_bytes(&d, &ws) == NEPTUNE_OK && ws > 0, "decode: workspace");
  expect(neptune_decode_splitk(&d, fake, fake, fake, nullptr, nullptr, fake, nullptr, fake, 16,
                               nullptr) == NEPTUNE_ERR_WORKSPACE_TOO_SMALL,
         "decode: workspace too small");
  neptune_decode_desc fp8 = d;
  fp8.kv_dtype = NEPTUNE_DTYPE_FP8_E4M3;
  expect(neptune_decode_splitk(&fp8, fake, fake, fake, nullptr, nullptr, fake, nullptr, fake, ws,
                               nullptr) == NEPTUNE_ERR_INVALID_ARGUMENT,
         "decode: fp8 without scales");
  neptune_decode_desc big = decode_desc(64, 64, 8, 64 * 4096, 64);
  expect(neptune_decode_splitk_noalloc(&big, fake, fake, fake, nullptr, nullptr, fake, nullptr,
                                       nullptr) == NEPTUNE_ERR_WORKSPACE_TOO_SMALL,
         "decode_noalloc: past the static scratch");
  neptune_scan_desc s = {1, 64, 0, 16, NEPTUNE_DTYPE_BF16, 1};
  expect(neptune_selective_scan_fwd(&s, fake, fake, (const float *)fake, fake, fake, nullptr,
                                    nullptr, nullptr, fake, nullptr) ==
             NEPTUNE_ERR_INVALID_ARGUMENT, "scan: seq_len 0");
  s.seq_len = 128;
  expect(neptune_selective_scan_fwd(&s, fake, fake, (const float *)fake, fake, fake, nullptr,
                                    nullptr, nullptr, fake, nullptr) ==
             NEPTUNE_ERR_INVALID_ARGUMENT &&
             std::string(neptune_last_error()) == "selective_scan: y overlaps u",
         "scan: y overlapping u");

  const int devices = neptune_device_count();
  if (devices == 0) {
    expect(neptune_attn_fwd(&a, fake, fake, fake, fake, nullptr, nullptr) ==
               NEPTUNE_ERR_NO_DEVICE, "attn: no device");
    expect(neptune_decode_splitk_noalloc(&d, fake, fake, fake, nullptr, nullptr, fake, nullptr,
                                         nullptr) == NEPTUNE_ERR_NO_DEVICE,
           "decode_noalloc: no device");
  }
  std::printf("validate: %s (%d devices)\n", g_failures ? "FAILED" : "ok", devices);
  return g_failures ? 1 : 0;
}

int run_attn(const std::string &dir) {
  auto m = read_meta(dir);
  neptune_attn_desc a = attn_desc((int64_t)m["batch"], (int64_t)m["heads_q"],
                                  (int64_t)m["heads_kv"], (int64_t)m["seq_q"],
                                  (int64_t)m["seq_kv"], 128);
  a.causal = (int32_t)m["causal"];
  const auto q = read_array<uint16_t>(dir + "/q.bin"), k = read_array<uint16_t>(dir + "/k.bin"),
             v = read_array<uint16_t>(dir + "/v.bin");
  const auto want_o = read_array<float>(dir + "/o.bin"),
             want_lse = read_array<float>(dir + "/lse.bin");
  DeviceBuffer dq(q), dk(k), dv(v), dout(q.size() * 2), dlse(want_lse.size() * 4);
  hipStream_t stream;
  if (!hip_ok(hipStreamCreate(&stream), "stream")) return 1;
  const neptune_status st =
      neptune_attn_fwd(&a, dq.ptr, dk.ptr, dv.ptr, dout.ptr, (float *)dlse.ptr, stream);
  expect(st == NEPTUNE_OK, "attn_fwd status");
  hip_ok(hipStreamSynchronize(stream), "sync");
  (void)hipStreamDestroy(stream);
  const double eo = max_err_bf16(dout.to_host<uint16_t>(), want_o);
  const double el = max_err_f32(dlse.to_host<float>(), want_lse);
  expect(eo <= m["tol"], "attn: output within tolerance");
  expect(el <= 1e-3, "attn: lse within 1e-3");
  std::printf("attn: %s max|o-ref|=%.3e max|lse-ref|=%.3e\n", g_failures ? "FAILED" : "ok", eo,
              el);
  return g_failures ? 1 : 0;
}

int run_decode(const std::string &dir) {
  auto m = read_meta(dir);
  neptune_decode_desc d = decode_desc((int64_t)m["batch"], (int64_t)m["heads_q"],
                                      (int64_t)m["heads_kv"], (int64_t)m["seq_kv"],
                                      (int64_t)m["num_splits"]);
  const auto q = read_array<uint16_t>(dir + "/q.bin"), k = read_array<uint16_t>(dir + "/k.bin"),
             v = read_array<uint16_t>(dir + "/v.bin");
  const auto want_o = read_array<float>(dir + "/o.bin"),
             want_lse = read_array<float>(dir + "/lse.bin");
  size_t ws_bytes = 0;
  expect(neptune_decode_workspace_bytes(&d, &ws_bytes) == NEPTUNE_OK, "workspace bytes");
  DeviceBuffer dq(q), dk(k), dv(v), ws(ws_bytes), o1(q.size() * 2), o2(q.size() * 2),
      l1(want_lse.size() * 4), l2(want_lse.size() * 4);
  expect(neptune_decode_splitk(&d, dq.ptr, dk.ptr, dv.ptr, nullptr, nullptr, o1.ptr,
                               (float *)l1.ptr, ws.ptr, ws_bytes, nullptr) == NEPTUNE_OK,
         "decode_splitk status");
  expect(neptune_decode_splitk_noalloc(&d, dq.ptr, dk.ptr, dv.ptr, nullptr, nullptr, o2.ptr,
                                       (float *)l2.ptr, nullptr) == NEPTUNE_OK,
         "decode_splitk_noalloc status");
  hip_ok(hipDeviceSynchronize(), "sync");
  const auto got1 = o1.to_host<uint16_t>(), got2 = o2.to_host<uint16_t>();
  const auto lse1 = l1.to_host<float>(), lse2 = l2.to_host<float>();
  double ref_max = 0.0;
  for (float x : want_o) ref_max = std::fmax(ref_max, std::fabs((double)x));
  const double eo = max_err_bf16(got1, want_o), el = max_err_f32(lse1, want_lse);
  expect(eo <= m["tol"] && eo <= m["tol"] * ref_max, "decode: output within tolerance");
  expect(el <= 1e-3, "decode: lse within 1e-3");
  expect(got1 == got2 && std::memcmp(lse1.data(), lse2.data(), lse1.size() * 4) == 0,
         "decode: noalloc bit-identical to the workspace entry point");
  std::printf("decode: %s max|o-ref|=%.3e (max|ref| %.3e) max|lse-ref|=%.3e\n",
              g_failures ? "FAILED" : "ok", eo, ref_max, el);
  return g_failures ? 1 : 0;
}

int run_fp8(const std::string &dir) {
  auto m = read_meta(dir);
  neptune_decode_desc d = decode_desc((int64_t)m["batch"], (int64_t)m["heads_q"],
                                      (int64_t)m["heads_kv"], (int64_t)m["seq_kv"],
                                      (int64_t)m["num_splits"]);
  d.kv_dtype = NEPTUNE_DTYPE_FP8_E4M3;
  d.scale_block = (int64_t)m["scale_block"];
  const auto q = read_array<uint16_t>(dir + "/q.bin");
  const auto k = read_array<uint8_t>(dir + "/k.bin"), v = read_array<uint8_t>(dir + "/v.bin");
  const auto ks = read_array<float>(dir + "/k_scale.bin"),
             vs = read_array<float>(dir + "/v_scale.bin");
  const auto want_o = read_array<float>(dir + "/o.bin"),
             want_lse = read_array<float>(dir + "/lse.bin");
  size_t ws_bytes = 0;
  expect(neptune_decode_workspace_bytes(&d, &ws_bytes) == NEPTUNE_OK, "fp8: workspace bytes");
  DeviceBuffer dq(q), dk(k), dv(v), dks(ks), dvs(vs), ws(ws_bytes), o1(q.size() * 2),
      o2(q.size() * 2), l1(want_lse.size() * 4), l2(want_lse.size() * 4);
  expect(neptune_decode_splitk(&d, dq.ptr, dk.ptr, dv.ptr, (const float *)dks.ptr,
                               (const float *)dvs.ptr, o1.ptr, (float *)l1.ptr, ws.ptr, ws_bytes,
                               nullptr) == NEPTUNE_OK,
         "fp8: decode_splitk status");
  expect(neptune_decode_splitk_noalloc(&d, dq.ptr, dk.ptr, dv.ptr, (const float *)dks.ptr,
                                       (const float *)dvs.ptr, o2.ptr, (float *)l2.ptr,
                                       nullptr) == NEPTUNE_OK,
         "fp8: decode_splitk_noalloc status");
  hip_ok(hipDeviceSynchronize(), "sync");
  const auto got1 = o1.to_host<uint16_t>(), got2 = o2.to_host<uint16_t>();
  const auto lse1 = l1.to_host<float>(), lse2 = l2.to_host<float>();
  double ref_max = 0.0;
  for (float x : want_o) ref_max = std::fmax(ref_max, std::fabs((double)x));
  const double eo = max_err_bf16(got1, want_o), el = max_err_f32(lse1, want_lse);
  expect(eo <= m["tol"] && eo <= m["tol"] * ref_max, "fp8: output within tolerance");
  expect(el <= 1e-3, "fp8: lse within 1e-3");
  expect(got1 == got2 && std::memcmp(lse1.data(), lse2.data(), lse1.size() * 4) == 0,
         "fp8: noalloc bit-identical to the workspace entry point");
  std::printf("fp8: %s max|o-ref|=%.3e (max|ref| %.3e) max|lse-ref|=%.3e\n",
              g_failures ? "FAILED" : "ok", eo, ref_max, el);
  return g_failures ? 1 : 0;
}

int run_scan(const std::string &dir) {
  auto m = read_meta(dir);
  neptune_scan_desc sd;
  std::memset(&sd, 0, sizeof sd);
  sd.batch = (int64_t)m["batch"];
  sd.dim = (int64_t)m["dim"];
  sd.seq_len = (int64_t)m["seq_len"];
  sd.d_state = (int64_t)m["d_state"];
  sd.io_dtype = NEPTUNE_DTYPE_BF16;
  sd.delta_softplus = 1;
  const auto u = read_array<uint16_t>(dir + "/u.bin"), dr = read_array<uint16_t>(dir + "/delta.bin"),
             Bm = read_array<uint16_t>(dir + "/B.bin"), Cm = read_array<uint16_t>(dir + "/C.bin"),
             z = read_array<uint16_t>(dir + "/z.bin");
  const auto A = read_array<float>(dir + "/A.bin"), D = read_array<float>(dir + "/D.bin"),
             bias = read_array<float>(dir + "/delta_bias.bin"),
             want = read_array<float>(dir + "/y.bin");
  DeviceBuffer du(u), ddr(dr), dB(Bm), dC(Cm), dz(z), dA(A), dD(D), dbias(bias),
      dy(u.size() * 2);
  expect(neptune_selective_scan_fwd(&sd, du.ptr, ddr.ptr, (const float *)dA.ptr, dB.ptr, dC.ptr,
                                    (const float *)dD.ptr, dz.ptr, (const float *)dbias.ptr,
                                    dy.ptr, nullptr) == NEPTUNE_OK,
         "scan: status");
  hip_ok(hipDeviceSynchronize(), "sync");
  const auto got = dy.to_host<uint16_t>();
  // |a - b| <= 2e-2 * max(1, |ref|), elementwise
  double worst = 0.0;
  for (size_t i = 0; i < want.size(); ++i) {
    const double err = std::fabs((double)bf16_to_f32(got[i]) - (double)want[i]);
    worst = std::fmax(worst, err / std::fmax(1.0, std::fabs((double)want[i])));
  }
  expect(worst <= 2e-2, "scan: y within 2e-2 * max(1, |ref|)");
  std::printf("scan: %s max |y-ref| / max(1,|ref|) = %.3e\n", g_failures ? "FAILED" : "ok",
              worst);
  return g_failures ? 1 : 0;
}

}  // namespace

int main(int argc, char **argv) {
  const std::string mode = argc > 1 ? argv[1] : "";
  if (mode == "validate") return run_validate();
  if (mode == "attn" && argc > 2) return run_attn(argv[2]);
  if (mode == "decode" && argc > 2) return run_decode(argv[2]);
  if (mode == "fp8" && argc > 2) return run_fp8(argv[2]);
  if (mode == "scan" && argc > 2) return run_scan(argv[2]);
  std::fprintf(stderr, "usage: %s validate | attn DIR | decode DIR | fp8 DIR | scan DIR\n",
               argv[0]);
  return 2;
}
