function flatmv_d(loss, lossd, a, ad, x, xd, y, yd, i_m, i_n)
    for idx = 1:i_m * i_n
        i = div(idx - 1, i_n) + 1
        j = mod(idx - 1, i_n) + 1
        yd[i] = yd[i] + (ad[idx] * x[j] + a[idx] * xd[j])
        y[i] = y[i] + a[idx] * x[j]
    end
    for k = 1:i_m
        lossd[1] = lossd[1] + 2 * y[k] * yd[k]
        loss[1] = loss[1] + y[k] ^ 2
    end
    return nothing
end

function flatmv(loss, a, x, y, i_m, i_n)
    for idx = 1:i_m * i_n
        i = div(idx - 1, i_n) + 1
        j = mod(idx - 1, i_n) + 1
        y[i] = y[i] + a[idx] * x[j]
    end
    for k = 1:i_m
        loss[1] = loss[1] + y[k] ^ 2
    end
    return nothing
end
