// gguf.cpp -- reads a GGUF model file (memory-mapped, host only) and finds
// the tensors and metadata of its MoE FFN blocks, the part of TIE's model
// loading (gguf_model_parse / gguf_model_map_weights, gguf.c:892-1030;
// model_load_tensor, model.c:198-235) that the GPU block needs.
//
// GGUF (v2/v3): magic "GGUF", version u32, tensor count u64, metadata count
// u64; metadata entries (key string, value type u32, value); tensor infos
// (name string, n_dims u32, dims u64[n], type u32, offset u64); tensor data
// at the first multiple of general.alignment (default 32) after the infos.
// Strings are a u64 length and bytes.
#include <fcntl.h>
#include <stdint.h>
#include <string.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <map>
#include <string>
#include <vector>

#include "../../include/tie_hip.h"
#include "gguf.h"

namespace tie {

int set_error(int code, const char *fmt, ...);

namespace {

struct Reader {
	const uint8_t *p, *end;
	bool ok = true;
	template <typename V> V get()
	{
		V v{};
		if (p + sizeof(V) > end) {
			ok = false;
			return v;
		}
		memcpy(&v, p, sizeof(V));
		p += sizeof(V);
		return v;
	}
	std::string str()
	{
		const uint64_t n = get<uint64_t>();
		if (!ok || n > (uint64_t)(end - p)) {
			ok = false;
			return std::string();
		}
		std::string s((const char *)p, (size_t)n);
		p += n;
		return s;
	}
};

// size in bytes of one scalar metadata value of type t (0: not a scalar)
size_t scalar_size(uint32_t t)
{
	switch (t) {
	case 0: case 1: case 7: return 1; // u8, i8, bool
	case 2: case 3: return 2;         // u16, i16
	case 4: case 5: case 6: return 4; // u32, i32, f32
	case 10: case 11: case 12: return 8; // u64, i64, f64
	default: return 0;
	}
}

bool skip_value(Reader &r, uint32_t t)
{
	if (t == 8) {
		r.str();
		return r.ok;
	}
	if (t == 9) {
		const uint32_t et = r.get<uint32_t>();
		const uint64_t n = r.get<uint64_t>();
		for (uint64_t i = 0; i < n && r.ok; i++)
			if (!skip_value(r, et))
				return false;
		return r.ok;
	}
	const size_t s = scalar_size(t);
	if (!s || r.p + s > r.end)
		return r.ok = false;
	r.p += s;
	return true;
}

} // namespace

GGUFFile::~GGUFFile()
{
	if (map && map != MAP_FAILED)
		munmap(map, size);
}

int GGUFFile::open(const char *path)
{
	const int fd = ::open(path, O_RDONLY);
	if (fd < 0)
		return set_error(TIE_HIP_EINVAL, "cannot open %s", path);
	struct stat st;
	if (fstat(fd, &st) != 0 || st.st_size < 24) {
		::close(fd);
		return set_error(TIE_HIP_EINVAL, "%s: not a GGUF file (size)", path);
	}
	size = (size_t)st.st_size;
	map = mmap(nullptr, size, PROT_READ, MAP_PRIVATE, fd, 0);
	::close(fd);
	if (map == MAP_FAILED) {
		map = nullptr;
		return set_error(TIE_HIP_EINVAL, "%s: mmap failed", path);
	}
	Reader r{(const uint8_t *)map, (const uint8_t *)map + size};
	if (r.get<uint32_t>() != 0x46554747u) // "GGUF"
		return set_error(TIE_HIP_EINVAL, "%s: bad magic", path);
	const uint32_t version = r.get<uint32_t>();
	if (version < 2 || version > 3)
		return set_error(TIE_HIP_EINVAL, "%s: GGUF version %u unsupported (2, 3)", path, version);
	const uint64_t n_tensors = r.get<uint64_t>(), n_kv = r.get<uint64_t>();
	uint64_t alignment = 32;
	for (uint64_t i = 0; i < n_kv && r.ok; i++) {
		const std::string key = r.str();
		const uint32_t t = r.get<uint32_t>();
		if (!r.ok)
			break;
		if (t == 8) {
			strs[key] = r.str();
			continue;
		}
		const size_t s = scalar_size(t);
		if (s) {
			Meta m;
			m.type = t;
			if (r.p + s > r.end) {
				r.ok = false;
				break;
			}
			memcpy(&m.raw, r.p, s);
			r.p += s;
			nums[key] = m;
			if (key == "general.alignment")
				alignment = m.as_u64();
			continue;
		}
		if (!skip_value(r, t))
			break;
	}
	if (!r.ok)
		return set_error(TIE_HIP_EINVAL, "%s: truncated metadata", path);
	if (alignment == 0 || (alignment & (alignment - 1)))
		return set_error(TIE_HIP_EINVAL, "%s: bad general.alignment %llu", path, (unsigned long long)alignment);
	for (uint64_t i = 0; i < n_tensors && r.ok; i++) {
		GGUFTensor t;
		const std::string name = r.str();
		t.n_dims = r.get<uint32_t>();
		if (t.n_dims > 4) {
			r.ok = false;
			break;
		}
		for (uint32_t j = 0; j < t.n_dims; j++)
			t.ne[j] = r.get<uint64_t>();
		t.type = r.get<uint32_t>();
		t.offset = r.get<uint64_t>();
		tensors[name] = t;
	}
	if (!r.ok)
		return set_error(TIE_HIP_EINVAL, "%s: truncated tensor infos", path);
	const uint64_t head = (uint64_t)(r.p - (const uint8_t *)map);
	data_offset = (head + alignment - 1) & ~(alignment - 1);
	for (auto &kv : tensors) {
		GGUFTensor &t = kv.second;
		uint64_t n = 1;
		for (uint32_t j = 0; j < t.n_dims; j++)
			n *= t.ne[j];
		// tensors of types the MoE path never reads (Q8_0 embeddings, F16
		// attention, ...) keep bytes = 0; the loader refuses them only if
		// it needs them
		t.bytes = tensor_bytes(t.type, n);
		if (data_offset + t.offset + t.bytes > size)
			return set_error(TIE_HIP_EINVAL, "%s: tensor %s extends past the end of the file", path,
					 kv.first.c_str());
		t.data = (const uint8_t *)map + data_offset + t.offset;
	}
	return TIE_HIP_OK;
}

uint64_t GGUFFile::tensor_bytes(uint32_t type, uint64_t n)
{
	switch (type) {
	case TIE_GGML_F32: return 4 * n;
	case TIE_GGML_BF16: return 2 * n;
	case 1: return 2 * n; // F16
	case TIE_GGML_Q4_K: return n % 256 ? 0 : n / 256 * 144;
	case TIE_GGML_Q6_K: return n % 256 ? 0 : n / 256 * 210;
	default: return 0; // types the MoE path does not read
	}
}

bool GGUFFile::num(const std::string &key, uint64_t &v) const
{
	auto it = nums.find(key);
	if (it == nums.end())
		return false;
	v = it->second.as_u64();
	return true;
}

bool GGUFFile::f32(const std::string &key, float &v) const
{
	auto it = nums.find(key);
	if (it == nums.end())
		return false;
	v = it->second.as_f32();
	return true;
}

const GGUFTensor *GGUFFile::tensor(const std::string &name) const
{
	auto it = tensors.find(name);
	return it == tensors.end() ? nullptr : &it->second;
}

// The MoE shape of the file (arch.* metadata as model_qwen3.c:57-59 and
// model_lfm2.c:49-64 read it), or an error if it has no MoE FFN.
int GGUFFile::moe_info(tie_hip_model_info &info) const
{
	memset(&info, 0, sizeof info);
	auto a = strs.find("general.architecture");
	if (a == strs.end())
		return set_error(TIE_HIP_EINVAL, "no general.architecture");
	const std::string arch = a->second;
	snprintf(info.architecture, sizeof info.architecture, "%s", arch.c_str());
	uint64_t d = 0, E = 0, k = 0, F = 0, L = 0, lead = 0;
	if (!num(arch + ".embedding_length", d) || !num(arch + ".block_count", L) || !num(arch + ".expert_count", E) ||
	    !num(arch + ".expert_used_count", k) || !num(arch + ".expert_feed_forward_length", F))
		return set_error(TIE_HIP_EINVAL, "%s: missing MoE metadata (embedding_length, block_count, expert_count, "
				 "expert_used_count, expert_feed_forward_length)", arch.c_str());
	num(arch + ".leading_dense_block_count", lead);
	float eps = 1e-6f;
	f32(arch + ".attention.layer_norm_rms_epsilon", eps);
	info.d = (int)d;
	info.F = (int)F;
	info.E = (int)E;
	info.k = (int)k;
	info.n_layers = (int)L;
	info.first_moe_layer = (int)lead;
	info.norm_eps = eps;
	// LFM2's MoE routes by sigmoid (model_lfm2.c:437-467), Qwen3's by softmax
	info.routing = arch.find("lfm2") != std::string::npos ? TIE_HIP_ROUTE_SIGMOID : TIE_HIP_ROUTE_SOFTMAX;
	return TIE_HIP_OK;
}

} // namespace tie

extern "C" int tie_hip_gguf_inspect(const char *path, tie_hip_model_info *info)
{
	if (!path || !info)
		return tie::set_error(TIE_HIP_EINVAL, "null argument");
	tie::GGUFFile f;
	int rc = f.open(path);
	if (rc)
		return rc;
	return f.moe_info(*info);
}

extern "C" int tie_hip_gguf_tensor_info(const char *path, const char *name, int *type, uint64_t ne[4],
					uint64_t *file_offset, uint64_t *bytes)
{
	if (!path)
		return tie::set_error(TIE_HIP_EINVAL, "null path");
	tie::GGUFFile f;
	int rc = f.open(path);
	if (rc)
		return rc;
	if (!name)
		return (int)f.tensors.size();
	const tie::GGUFTensor *t = f.tensor(name);
	if (!t)
		return tie::set_error(TIE_HIP_EINVAL, "%s: no tensor %s", path, name);
	if (type)
		*type = (int)t->type;
	if (ne)
		for (int j = 0; j < 4; j++)
			ne[j] = t->ne[j];
	if (file_offset)
		*file_offset = f.data_offset + t->offset;
	if (bytes)
		*bytes = t->bytes;
	return (int)f.tensors.size();
}
